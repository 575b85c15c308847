/*
 * tbhip_bench.h -- measurement entry points of libtbhip.so.  They have no
 * counterpart in the reference and no place in a binding of it; bench.py uses
 * them to time the decoder's graph replays and a plain streaming read of the
 * GEMVs' byte counts.  The product header (tbhip.h) does not include this file.
 */
#ifndef TBHIP_BENCH_H
#define TBHIP_BENCH_H

#include "tbhip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Benchmark helper (no reference counterpart): n_steps greedy steps from
 * (first_token, offset) as back-to-back graph replays, timed with HIP events on
 * the decoder's stream. */
TB_API int tb_decoder_time_greedy(tb_decoder *d, int64_t first_token, int64_t offset,
                                  int64_t n_steps, float *ms_out);

/* Measurement aid (no reference counterpart): one plain streaming read of
 * device memory, for the benchmark to set each GEMV's bandwidth beside what a
 * read of the same byte count reaches on this GPU.  `blocks` blocks of 256
 * threads each read a contiguous share of buf (16-byte aligned) in passes of
 * `loads` (4, 8 or 16) non-temporal 16-byte loads per thread (the last pass
 * masked), and write one xor-folded word per thread to out[blocks * 256]
 * (device memory).  bytes is rounded down to a multiple of 16; the bytes read
 * go to *bytes_read (host). */
TB_API int tb_read_probe(const void *buf, int64_t bytes, int64_t blocks, int64_t loads,
                         uint32_t *out, int64_t *bytes_read, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TBHIP_BENCH_H */
