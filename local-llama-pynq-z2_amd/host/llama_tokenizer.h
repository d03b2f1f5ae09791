/* llama2.c tokenizer of runq (tokenizer.bin: int max_token_length, then per id: float score, int length,
 * bytes; runq.c:638-662), for the runq host's text prompts and output.
 *
 * encode follows runq.c:705-823: optional BOS (1), a dummy-prefix " " token when the text is not empty,
 * one token per UTF-8 character found in the vocabulary or one per byte (id byte + 3) otherwise, then
 * repeated merges of the adjacent pair whose concatenation is the vocabulary entry of highest score (the
 * first such pair on equal scores; only scores above -1e10 merge), optional EOS (2).  decode follows
 * runq.c:671-684 (a leading space is dropped after BOS; "<0xHH>" pieces are raw bytes) and
 * llama_print_piece runq.c:686-697 (a single non-printable, non-space byte is not printed). */
#pragma once
#include <stdio.h>

typedef struct LlamaTokenizer LlamaTokenizer;

LlamaTokenizer *llama_tok_load(const char *path, int vocab_size); /* NULL, with a message, on failure */
void llama_tok_free(LlamaTokenizer *t);

/* tokens needs room for strlen(text) + 3 ids; returns 0, or -1 for a NULL text */
int llama_encode(LlamaTokenizer *t, const char *text, int bos, int eos, int *tokens, int *n_tokens);
const char *llama_decode(LlamaTokenizer *t, int prev_token, int token); /* NULL for an id out of range */
void llama_print_piece(const char *piece, FILE *f);
