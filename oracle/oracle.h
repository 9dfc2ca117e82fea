/*
 * oracle.h -- CPU restatement of the reference's graph-restore (LOAD) path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline) -- never as part of the product.
 *
 * Built with g++ from oracle.cpp alone; it shares no code with the product
 * (own CRC, own format reader, own relocation search) so that a mistake in
 * one is not silently repeated in the other.
 *
 * What each function follows is cited in oracle.cpp.  How each is pinned
 * (golden fixtures, textbook check values, invariants, brute force) is in
 * the header comment of oracle.cpp.
 */
#ifndef FDY_ORACLE_H
#define FDY_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_result orc_result;

typedef struct orc_override {
  uint32_t word;
  uint32_t node;
  uint64_t value;
} orc_override;

const char* orc_last_error(void);

/* CRC-64/XZ (reflected poly 0x42F0E1EBA9EA3693, init/xorout ~0): the hash of
 * csrc/hook.cpp:315-321.  Plain byte-at-a-time table walk. */
uint64_t orc_crc64(const uint8_t* data, uint64_t n);

/* Saved topology key (include/BinaryGraphFormat.h:274-278) and the key the
 * LOAD fallback recomputes from nodes (csrc/CUDAGraphParallel.cpp:1798-1841).
 * Return the key length; copy at most cap bytes. <0 on a bad image. */
int64_t orc_topology_key_saved(const uint8_t* image, uint64_t size, char* buf, uint64_t cap);
int64_t orc_topology_key_recomputed(const uint8_t* image, uint64_t size, char* buf, uint64_t cap);

/* Grouping by key string (csrc/CUDAGraphParallel.cpp:1788-1851):
 * template_for[i] = lowest index with the same key (itself for templates). */
int orc_group_by_keys(const char* const* keys, const uint64_t* lens, uint32_t n, uint32_t* template_for);

/* Grouping from a graph_manifest.json text (csrc/CUDAGraphParallel.cpp:1727-1786).
 * names[i] = file name of graph i.  out[i] = the template of a member, or
 * UINT32_MAX for a graph that builds its own exec (a template, or a graph no
 * group lists), as template_for = SIZE_MAX there.  Returns 0, or -1 if the
 * manifest does not parse (the reference then falls back to keys). */
int orc_group_manifest(const char* manifest, uint64_t len, const char* const* names, uint32_t n,
                       uint32_t* out);

/* Effective launch attributes of kernel node `node`, merged as
 * prepare_on_demand_graph_binary does (csrc/CUDAGraphParallel.cpp:1211-1389):
 * out[17] = has_cluster, cx, cy, cz, has_pref, px, py, pz, sched, coop, prio,
 * msd, has_map, map_default, map_remote, has_carveout, carveout.  -1 if the
 * node is not a kernel node or the image is bad. */
int orc_effective_attrs(const uint8_t* image, uint64_t size, uint32_t node, int32_t* out);

/* Test hook: plant mistake m (1..6) in the attribute merge, 0 to remove it.
 * 1 common wins over per-node, 2 negative per-node scalars override,
 * 3 required cluster ignored, 4 per-node attrs replace common wholesale,
 * 5 common attrs ignored, 6 required zero dims stay 0.  Not thread-safe;
 * for the tests that show the attribute fixtures pin the merge. */
void orc_set_mutation(int m);

/* Per-param byte extraction of one kernel node (csrc/CUDAGraphParallel.cpp:1391-1409):
 * writes the node's params back-to-back into out (or the arg buffer for
 * extra-style nodes).  Returns bytes written, -1 on bounds error. */
int64_t orc_extract_node_params(const uint8_t* image, uint64_t size, uint32_t node, uint8_t* out, uint64_t cap);

/* The whole restore on the CPU.  template_of may be NULL (group by keys). */
int orc_restore(const uint8_t* const* images, const uint64_t* sizes, uint32_t n, const uint64_t* lo,
                const uint64_t* hi, const uint64_t* new_lo, uint64_t n_iv, uint32_t policy,
                const uint32_t* template_of, uint32_t num_threads, orc_result** out);
void orc_free(orc_result* r);

int orc_digests(const orc_result* r, uint64_t* out /* 4n */);
int orc_groups(const orc_result* r, uint32_t* out /* n */);
int orc_status(const orc_result* r, uint32_t* out /* n */);
int orc_override_offsets(const orc_result* r, uint64_t* out /* n+1 */);
int64_t orc_overrides(const orc_result* r, uint32_t g, orc_override* out, uint64_t cap);
int64_t orc_node_flags(const orc_result* r, uint32_t g, uint8_t* out, uint64_t cap);
int64_t orc_node_words(const orc_result* r, uint32_t g, uint32_t* out, uint64_t cap);
int64_t orc_param_image(const orc_result* r, uint32_t g, uint64_t* out, uint64_t cap);
int64_t orc_node_pointers(const orc_result* r, uint32_t g, uint64_t* out, uint64_t cap);
uint64_t orc_total_param_bytes(const orc_result* r);

/* Switch simulation: per group, the live image and node sources. */
int orc_switch(orc_result* r, uint32_t g);
int64_t orc_live(const orc_result* r, uint32_t template_graph, uint64_t* words, uint64_t cap,
                 uint32_t* node_src, uint64_t node_cap, uint32_t* current);

/* One word, and packed words (value semantics of the relocation table). */
uint64_t orc_relocate_word(uint64_t w, const uint64_t* lo, const uint64_t* hi, const uint64_t* new_lo,
                           uint64_t n, uint32_t policy);
int orc_relocate_words(const uint64_t* in, uint64_t* out, uint64_t n_words, const uint64_t* lo,
                       const uint64_t* hi, const uint64_t* new_lo, uint64_t n, uint32_t policy,
                       uint32_t num_threads);

/* Replay of one graph's allocator events (csrc/hook.cpp:3394-3492) on a
 * region whose cursor is *cursor (absolute address), with the placement rule
 * of cuMemAlloc_v2 (csrc/hook.cpp:2272-2291, 2424) and the reserve carve
 * (2705-2721).  Saved addresses are offsets from saved_base, placements
 * offsets from base.  Writes (saved lo, saved hi, new lo) per alloc or
 * reserve into out (3 per placement, at most cap placements) and advances
 * *cursor.  Returns the number of placements, -1 if the text does not parse,
 * -2 on a mismatch (the reference aborts), -3 if the region is too small. */
int64_t orc_region_replay(const char* json, uint64_t len, uint64_t saved_base, uint64_t base, uint64_t size,
                          uint64_t* cursor, uint64_t* out, uint64_t cap);

/* The reference's CPU LOAD data work, restated (csrc/CUDAGraphParallel.cpp):
 * read files (1583-1620), build key strings and group (1788-1851), and per
 * node the prep of prepare_on_demand_graph_binary (1288-1473) minus driver
 * calls: name string + registry lookup, one vector + memcpy per param.
 * Runs `reps` times on a SimpleThreadPool clone of num_threads; returns the
 * median wall time in ms, or <0 on error.  Driver calls skipped are
 * counted into *driver_calls. */
double orc_reference_load_ms(const char* const* paths, uint32_t n, uint32_t num_threads, uint32_t reps,
                             uint64_t* driver_calls);

#ifdef __cplusplus
}
#endif

#endif
