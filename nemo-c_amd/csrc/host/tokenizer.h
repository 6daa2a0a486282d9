/* SentencePiece piece -> text (after the hot path; token ids are the parity object).
 * Same behaviour as the reference's src/tokenizer.c:19-50: U+2581 becomes a space; <unk>, <pad>,
 * <s>, </s> and <xx-YY> language tags produce no text. */
#ifndef NEMO_TOKENIZER_H
#define NEMO_TOKENIZER_H
#include "json.h"

typedef struct {
    char **piece;
    int n;
} vocab_t;

int vocab_load(const jn_t *arr, vocab_t *v);
void vocab_release(vocab_t *v);
int piece_is_lang_tag(const char *p);
int piece_is_special(const char *p);
char *piece_text(const vocab_t *v, int id); /* malloc'd; "" for specials and out-of-range ids */

#endif
