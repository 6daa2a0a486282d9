/* Plain-C wrappers of host bookkeeping for CPU tests (include/nemoasr_host.h). */
#include "nemoasr_host.h"
#include "encoder.h"
#include "tokenizer.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* state_out: [0] pending_n, [1] consumed, [2] emitted, [3] mel_cache_n, [4] closed (as ints) */
int nemo_enc_plan(int *plan, size_t pending_n, size_t consumed, size_t emitted, int mel_cache_n, int closed, int final,
                  int chunk_mel, int subsampling, int mel_cache, int *state_out) {
    enc_book_t b = { pending_n, consumed, emitted, mel_cache_n, closed };
    const enc_plan_t p = enc_plan_step(&b, final, chunk_mel, subsampling, mel_cache);
    const int v[8] = { p.ran, p.take, p.nwin, p.lo, p.hi, p.c, p.include_boundary, p.T3 };
    memcpy(plan, v, sizeof v);
    state_out[0] = (int)b.pending_n;
    state_out[1] = (int)b.consumed;
    state_out[2] = (int)b.emitted;
    state_out[3] = b.mel_cache_n;
    state_out[4] = b.closed;
    return p.ran;
}

int nemo_piece_text(const char *piece, size_t unused, char *out, size_t outlen) {
    (void)unused;
    char *pieces[1] = { (char *)piece };
    vocab_t v = { pieces, 1 };
    char *t = piece_text(&v, 0);
    const size_t n = strlen(t);
    if (n + 1 > outlen) { free(t); return -1; }
    memcpy(out, t, n + 1);
    free(t);
    return 0;
}
