/* Qwen2 / Qwen2.5 byte-level BPE tokenizer of the C hosts (text prompts in, token text out).
 *
 * Same interface and data file as the reference's qwen/tokenizer.h:1-20 (tok_load, tok_free, tok_encode,
 * tok_decode, tok_id, tok_vocab_size over a "QWTOK001" file written by tools/qwen_tok_export.py from Hugging
 * Face's tokenizer.json), so qwen.c's prompt code (qwen.c:778-797) links against it unchanged.  The ids are
 * those of Hugging Face `tokenizers` for Qwen2.5: added tokens split first (leftmost, then longest), NFC,
 * the Qwen2 pre-tokenizer regex, byte-level symbols, BPE merges by rank (leftmost on equal rank). */
#pragma once

typedef struct Tokenizer Tokenizer;

Tokenizer *tok_load(const char *path); /* NULL, with the reason on stderr, on failure */
void tok_free(Tokenizer *t);

/* ids of the UTF-8 text; allow_special != 0 turns added tokens written in the text ("<|im_start|>") into
 * their ids.  Returns the number of ids, or -1 when more than max_ids would be needed. */
int tok_encode(Tokenizer *t, const char *text, int allow_special, int *ids, int max_ids);

/* the raw bytes of one token (not NUL-terminated; *len gets the count), NULL for an unknown id */
const char *tok_decode(Tokenizer *t, int id, int *len);

int tok_id(Tokenizer *t, const char *added_token); /* id of an added token such as "<|im_end|>", or -1 */
int tok_vocab_size(Tokenizer *t);                  /* ids known: base vocabulary plus added tokens */
