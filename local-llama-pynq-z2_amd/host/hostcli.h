/* Shared piece of the C host programs qwen_hip and runq_hip: prompt-id parsing.
 * Decoding (argmax or the sampler) runs on the device inside the step graph. */
#pragma once
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int *parse_ids(const char *arg, int *n) { /* qwen.c:771-777 */
    int *ids = calloc(strlen(arg) / 2 + 2, sizeof(int));
    *n = 0;
    for (const char *c = arg; *c;) {
        char *end;
        long v = strtol(c, &end, 10);
        if (end == c || (*end && *end != ',') || v < 0) { fprintf(stderr, "bad --ids\n"); exit(EXIT_FAILURE); }
        ids[(*n)++] = (int)v;
        c = *end ? end + 1 : end;
    }
    return ids;
}
