/*
 * fdy_synth.h -- seeded synthetic `.cugraph` archives for tests and benchmarks.
 *
 * Every archive is produced through the same writer as a real SAVE
 * (csrc/BinaryGraphIO.cpp:15-371 layout), so the restore path reads exactly
 * what it would read from disk.  Randomness is SplitMix64 (Steele, Lea and
 * Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014);
 * each graph has its own stream, so graphs are generated in parallel and the
 * result does not depend on the thread count.
 *
 * Presets (fdy_synth_preset):
 *   1  64 graphs x 120 kernel nodes, one topology group, blobs 64-512 B,
 *      30% pointers in [0x7f0000000000, +4 GiB), 5% of words differ, one
 *      interval rebased to 0x7e0000000000.
 *   2  256 graphs (batch sizes 1,2,4..510) x 1200 kernel nodes (48 layers x 25),
 *      4 groups, blobs 32-1024 B in 1-16 params, 25% pointers into a 64 GiB
 *      region of 40k intervals, 3% of words differ.
 *   3  256 graphs x ~3000 nodes (85% kernel, 10% memset, 5% memcpy), 16 groups,
 *      blobs up to 4 KiB in 1-40 params, 10% of words differ in 64-256 B runs.
 *   4  words only: 1 GiB of packed words, 40% pointers, 2M intervals tiling
 *      200 GiB, 1% boundary pointers (lo, hi-1, hi, lo-1).
 *   5  1024 graphs x 5000 nodes in 32 groups, 1-8% of words differ per graph.
 * Every numeric field can be overridden after fdy_synth_preset().
 */
#ifndef FDY_SYNTH_H
#define FDY_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fdy_synth_params {
  uint32_t preset;
  uint32_t num_graphs;
  uint32_t num_groups;
  uint32_t nodes_per_graph;
  uint32_t min_blob_bytes;   /* per kernel node, multiple of 8 */
  uint32_t max_blob_bytes;
  uint32_t max_params;       /* a blob is split into 1..max_params params */
  uint32_t ragged;           /* 1: some params get sizes that are not multiples of 8 */
  uint32_t extra_style_pct;  /* % of kernel nodes whose params travel in an arg buffer */
  uint32_t memset_pct;       /* % of nodes that are memset nodes */
  uint32_t memcpy_pct;       /* % of nodes that are memcpy nodes */
  uint32_t event_pct;        /* % of nodes that are event record/wait pairs */
  uint32_t grid_bs_pct;      /* % of kernel nodes whose grid depends on the batch size */
  uint32_t layout_var_pct;   /* % of kernel nodes whose param layout changes with batch size */
  uint32_t run_min_bytes;    /* >0: differing words come in runs of this many bytes ... */
  uint32_t run_max_bytes;    /* ... up to this many */
  double pointer_frac;
  double diff_lo;            /* per-graph fraction of words that differ from the group base */
  double diff_hi;
  uint64_t seed;
  uint64_t region_base;
  uint64_t region_size;
  uint64_t new_base;
  uint32_t num_intervals;    /* 1 = uniform rebase of the whole region */
  uint32_t interval_granule; /* bytes; intervals tile the region at this granularity */
  uint64_t interval_min;     /* log-uniform sizes before the rescale */
  uint64_t interval_max;
  uint64_t num_words;        /* preset 4: packed words to generate */
  double boundary_frac;      /* preset 4: fraction of pointers on interval edges */
  uint64_t sink_hash;        /* nonzero: every kernel node names kernel "fdy_sink" of the code object
                                with this hash, and groups differ by a kernel/empty pattern in nodes
                                1..6 instead of by cluster dims (graphs a gfx950 group graph can build) */
  uint32_t diff_node_pct;    /* 0: differing words may fall in any kernel node; else only in this % of the
                                kernel nodes, the same ones in every graph of a group (arguments that
                                depend on the batch size live in a few kernels) */
  uint32_t pad_;
} fdy_synth_params;

typedef struct fdy_synth fdy_synth;

int fdy_synth_preset(uint32_t preset, fdy_synth_params* out);
/* Generate on `num_threads` host threads (0 = hardware concurrency). */
int fdy_synth_create(const fdy_synth_params* p, uint32_t num_threads, fdy_synth** out);
int fdy_synth_destroy(fdy_synth* s);
uint32_t fdy_synth_num_graphs(const fdy_synth* s);
int fdy_synth_image(const fdy_synth* s, uint32_t graph, const uint8_t** data, uint64_t* size);
int fdy_synth_batch_size(const fdy_synth* s, uint32_t graph, uint32_t* bs);
int fdy_synth_intervals(const fdy_synth* s, const uint64_t** lo, const uint64_t** hi, const uint64_t** new_lo,
                        uint64_t* n);
int fdy_synth_words(const fdy_synth* s, const uint64_t** words, uint64_t* n);
/* Writes graph_<i>.cugraph for every graph into `dir` (which must exist). */
int fdy_synth_write_dir(const fdy_synth* s, const char* dir);
/* n graph indices uniform over [0, num_graphs), from SplitMix64(seed). */
int fdy_synth_switch_sequence(uint64_t seed, uint32_t num_graphs, uint32_t n, uint32_t* out);
const char* fdy_synth_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FDY_SYNTH_H */
