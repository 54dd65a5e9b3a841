/*
 * Measurement probes used by bench.py (libmcq4_bench.so).  They are not part of
 * the drop-in library (libmcq4.so) and have no counterpart in the reference:
 * each measures one property of the machine that the decode and prefill
 * figures are read against.  Status codes as in mcq4.h (0 = OK); every probe is
 * enqueued on the given HIP stream and allocates nothing.
 */
#ifndef MCQ4_BENCH_H
#define MCQ4_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Plain streaming read of floor(bytes/16)*16 bytes at src (16-byte aligned):
 * 256-thread workgroups of 16 KiB each, non-temporal loads.  Writes *sink (a
 * device uint32) only if the XOR of a workgroup's data equals 0x9E3779B9. */
int mcqb_read_probe(const void *src, size_t bytes, uint32_t *sink, void *stream);

/* The same bytes read in the access pattern of a q4_0 weight [K/32][N][18]
 * split into tiles of tile_cols columns (18*tile_cols bytes per K row) and
 * ksplit K ranges: workgroup (t, s) of `waves` waves reads rows
 * [s*nb/ksplit, (s+1)*nb/ksplit) of tile t.  tile_cols * 18 must be a multiple
 * of 16 and divide N * 18; waves in {4, 8, 16}. */
int mcqb_read_tiles(const void *W, int64_t K, int64_t N, int tile_cols, int ksplit, int waves,
                    uint32_t *sink, void *stream);

/* Any row-piece pattern: rows of row_bytes bytes (a multiple of 16) split into
 * pieces of piece_bytes (a multiple of 16 that divides row_bytes) and ksplit row
 * ranges; workgroup (t, s) reads rows [s*rows/ksplit, (s+1)*rows/ksplit) of piece
 * column t.  The per-group INT4 weight [K/2][N] is rows = K/2, row_bytes = N. */
int mcqb_read_rows(const void *W, int64_t rows, int64_t row_bytes, int64_t piece_bytes, int ksplit, int waves,
                   uint32_t *sink, void *stream);

/* An empty kernel of grid x block threads (the per-launch floor). */
int mcqb_empty(int grid, int block, void *stream);

/* Shader clock under a dense MFMA load: 512 workgroups of 4 waves, `iters`
 * rounds of four v_mfma_f32_32x32x16_f16 chains on fresh pseudo-random
 * operands; per wave w, ticks[2w] = shader-clock ticks (s_memtime) and
 * ticks[2w+1] = 100 MHz real-time ticks of the loop (ticks: 4096 uint64). */
int mcqb_measure_sclk(uint64_t *ticks, int iters, void *stream);

/* Round trip of a returning 64-bit atomic add: `grid` one-wave workgroups each
 * run a dependent chain of `iters` atomics on their own word of p (64 words
 * apart; p holds grid*64 int64) and write the chain's 100 MHz ticks to
 * ticks[wg]. */
int mcqb_atomic_chain(int64_t *p, int iters, int grid, uint64_t *ticks, void *stream);

/* Store-to-load visibility between workgroups: 256 one-wave workgroups in
 * pairs (wg, wg + pair_stride) within blocks of 2*pair_stride; the first of a
 * pair stores a 64-bit word after a short delay, the second polls it (at most
 * `polls` loads).  store_mode: 0 plain, 1 agent-scope atomic store, 2
 * non-temporal; load_mode: 0 L1-coherent buffer load (sc0), 1 agent-scope
 * atomic load.  out[4*wg + {0,1,2,3}] = XCC id, store time, time the poll
 * ended (100 MHz ticks), 1 if the value was seen.  slots: 4096 zeroed uint64;
 * out: 1024 uint64. */
int mcqb_exchange(uint64_t *slots, uint64_t *out, int pair_stride, int store_mode, int load_mode,
                  int polls, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MCQ4_BENCH_H */
