/*
 * foundry_restore.h -- C ABI of the MI355X graph-restore (LOAD) data path.
 *
 * libfoundry_restore.so turns a set of `.cugraph` archives into restorable
 * graphs on one MI355X (gfx950).  Every data-parallel step runs as a
 * hand-written HIP kernel on the device; the host side only reads files,
 * validates section bounds and enqueues work.
 *
 * Conventions
 *   - Every call returns int: FDY_OK (0) or a negative FDY_E_* code.
 *     fdy_last_error() returns a message for the calling thread's last error.
 *     No C++ exception crosses this boundary.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Enqueueing calls are asynchronous; calls that return host arrays
 *     synchronize the stream they name and say so.
 *   - One fdy_archive is not safe for concurrent use from several threads;
 *     distinct archives are independent.
 *   - Arrays are caller-owned; device buffers are owned by the archive.
 *
 * Where the reference does this work (paths relative to the reference root):
 *   read .cugraph files          csrc/CUDAGraphParallel.cpp:1575-1620, csrc/BinaryGraphIO.cpp:710-737
 *   topology grouping            csrc/CUDAGraphParallel.cpp:1720-1851
 *   per-graph param materialise  csrc/CUDAGraphParallel.cpp:1192-1480 (prepare_on_demand_graph_binary)
 *   switch to another graph      csrc/CUDAGraph.cpp:330-461 (CUDAGraph::replay, on-demand branch)
 * The reference has no diff and no pointer relocation; their semantics are
 * defined here (see the comments on each call).
 */
#ifndef FOUNDRY_RESTORE_H
#define FOUNDRY_RESTORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define FDY_OK 0
#define FDY_E_INVALID (-1)  /* bad argument */
#define FDY_E_IO (-2)       /* file missing or unreadable */
#define FDY_E_FORMAT (-3)   /* not a valid .cugraph v1, or a section out of bounds */
#define FDY_E_HIP (-4)      /* a HIP runtime call failed (message carries hipError_t) */
#define FDY_E_NOMEM (-5)    /* host or device allocation failed */
#define FDY_E_RANGE (-6)    /* index out of range */
#define FDY_E_STATE (-7)    /* call out of order (e.g. results before fdy_restore) */
#define FDY_E_CAPACITY (-8) /* caller array too small; *_needed outputs say how big */
#define FDY_E_MISMATCH (-9) /* graph and template disagree in node count (reference: TORCH_CHECK), or a
                               replayed allocation lands elsewhere than it was saved */
#define FDY_E_NOT_FOUND (-10)   /* no code object with that hash, or no function of that name in it */
#define FDY_E_UNSUPPORTED (-11) /* a node, attribute or request with no gfx950 counterpart */

/* ---- relocation policy (fdy_archive_set_relocation / fdy_reloc_plan_create) ----
 * A word w is relocated by interval i = the last i with lo[i] <= w, if
 *   FDY_RELOC_HALF_OPEN:   w <  hi[i]   (one-past-end stays unchanged unless it is lo[i+1])
 *   FDY_RELOC_INCLUSIVE:   w <= hi[i]   (one-past-end moves with its interval)
 * and then w' = w - lo[i] + new_lo[i] (mod 2^64).  Otherwise w is unchanged. */
#define FDY_RELOC_HALF_OPEN 0u
#define FDY_RELOC_INCLUSIVE 1u

/* ---- per-node diff flags (fdy_get_node_flags) -------------------------- */
#define FDY_NODE_LAYOUT 0x01u  /* node type, param count or param sizes differ from the template */
#define FDY_NODE_DESC 0x02u    /* launch config / function / attributes / memset-memcpy fields differ */
#define FDY_NODE_RAGGED 0x04u  /* node has a param whose size is not a multiple of 8 */
#define FDY_NODE_TEMPLATE 0x08u

/* ---- per-graph status bits (fdy_get_graph_status) ---------------------- */
#define FDY_GRAPH_TYPE_MISMATCH 0x01u /* recomputed node-type digest differs from the template's */
#define FDY_GRAPH_BAD_PARAMS 0x02u    /* a param/arg/name range lies outside its section */
#define FDY_GRAPH_COLLISION 0x08u     /* a lower graph's key has an equal digest and length but other bytes
                                         (grouped apart all the same: groups follow the exact key bytes) */
#define FDY_GRAPH_NODE_COUNT 0x10u    /* node count differs from the template (switch refused) */
#define FDY_GRAPH_OVERFLOW 0x20u      /* param image larger than the capacity the sections allow */

/* One override: the word `word` of the template's param image takes `value`. */
typedef struct fdy_override {
  uint32_t word; /* template-image word index (node-major, params padded to 8 B) */
  uint32_t node; /* node index inside the graph */
  uint64_t value;
} fdy_override;

/* ---- restore scratch (fdy_archive_info.scratch) --------------------------
 * A restore keeps a bounded share of candidate words per diff sub-range
 * (continued in spill space shared by the sub-ranges of a 4096-word tile)
 * and a bounded override region per graph, and no ragged-word sources.  A
 * restore that runs out of either, or meets a node whose params are not
 * whole aligned words, is run again with what it lacked before any of its
 * results is read (the results are the same; the earlier run's time is
 * lost), and the archive keeps that layout for later restores.  Levels:
 *   0  768 candidates per 4096 words, an override record per 8 words
 *   1  2048 candidates per 4096 words, a record per 4 words
 *   2  a candidate and a record per word (cannot overflow) */
#define FDY_SCRATCH_LEVEL 0x3u   /* scratch level, 0..2 */
#define FDY_SCRATCH_RAGGED 0x4u  /* ragged-word sources held (one word per image word) */

typedef struct fdy_archive_info {
  uint32_t num_graphs;
  uint32_t num_groups;      /* valid after fdy_restore */
  uint64_t total_nodes;
  uint64_t total_param_bytes;  /* sum of kernel param sizes (+ extra arg buffers) */
  uint64_t total_words;        /* param-image words (valid after fdy_restore) */
  uint64_t total_overrides;    /* valid after fdy_restore */
  uint64_t file_bytes;         /* bytes of .cugraph images resident in HBM */
  uint64_t num_intervals;
  uint64_t device_bytes;       /* device memory the archive holds */
  uint32_t serving_layout;     /* 1 while in the serving layout (see fdy_group_graph_create) */
  uint32_t scratch;            /* FDY_SCRATCH_* bits: how the restore's scratch is laid out */
} fdy_archive_info;

typedef struct fdy_archive fdy_archive;
typedef struct fdy_reloc_plan fdy_reloc_plan;

const char* fdy_last_error(void);
const char* fdy_version(void);

/* Open `n` archives given by path.  A path ending in ".json" names the
 * sibling ".cugraph" (csrc/CUDAGraphParallel.cpp:1591-1594).  Where that
 * file is missing, shorter than a header or not a v1 header, the graph is
 * read from the JSON document at the path itself, as the reference then
 * parses it (1606-1617), converted with fdy_cugraph_from_json except that
 * its TOPOLOGY_KEY section holds the key the reference groups such a graph
 * by (fdy_load_topology_key: recomputed from the nodes when the document's
 * topology_key is missing or empty, 1796-1840).  Files are
 * read on min(num_threads, n) host threads (csrc/CUDAGraphParallel.cpp:
 * 1553,1584), validated, and copied to HBM in one transfer.  Replaces
 * Phase 1a. */
int fdy_archive_open(const char* const* paths, uint32_t n, uint32_t num_threads, fdy_archive** out);

/* The .cugraph v1 archive of one graph's JSON document (the object
 * CUDAGraph::save builds, csrc/CUDAGraph.cpp:1389-1491), byte for byte as
 * CUDAGraph::save_binary writes it (csrc/BinaryGraphIO.cpp:15-371).
 * *size_out receives the archive size; with out NULL or cap below that size
 * the call returns FDY_E_CAPACITY and writes nothing.  A document the
 * reference cannot serialise (a required member missing, a value of the
 * wrong type or out of its field's range, an unreadable value_hex pair) is
 * FDY_E_FORMAT, as are duplicate keys; a non-integer number inside
 * allocator_events or output_tensors is FDY_E_UNSUPPORTED.  No device
 * needed. */
int fdy_cugraph_from_json(const char* json, uint64_t len, uint8_t* out, uint64_t cap, uint64_t* size_out);
/* The key start_graph_builds groups a graph read from its JSON document by
 * (csrc/CUDAGraphParallel.cpp:1791-1841): the document's topology_key when
 * it is a non-empty string, else the key recomputed from its nodes (node
 * type strings joined by ','; a KernelNode gets ":C<x>_<y>_<z>" from its
 * kernel_node_attrs cluster dims, else the common attrs', else its
 * func_attrs' required_cluster_* fields, or ":0" when all are zero).  A
 * graph read from a .cugraph is grouped by its saved key as it stands.
 * The key's bytes (no NUL) go to out; *size_out receives its length, and
 * with out NULL or cap below it the call returns FDY_E_CAPACITY.  No device
 * needed. */
int fdy_load_topology_key(const char* json, uint64_t len, char* out, uint64_t cap, uint64_t* size_out);

/* fdy_cugraph_from_json into the file bin_path (CUDAGraph::save_binary;
 * CUDAGraph::save names it after the .json path, csrc/CUDAGraph.cpp:
 * 1494-1501).  FDY_E_IO when the file cannot be written, where the
 * reference prints a warning and returns. */
int fdy_cugraph_save_binary(const char* bin_path, const char* json, uint64_t len);

/* Same, from archive images already in host memory. */
int fdy_archive_open_images(const uint8_t* const* images, const uint64_t* sizes, uint32_t n,
                            fdy_archive** out);

int fdy_archive_close(fdy_archive* a);
/* Sizes and counts.  After fdy_restore this synchronizes the restore's stream. */
int fdy_archive_info_get(fdy_archive* a, fdy_archive_info* out);

/* Saved allocation intervals [lo, hi) -> new_lo, sorted by lo, non-overlapping.
 * n == 0 disables relocation (words pass through).  The interval model is the
 * allocator cursor of csrc/hook.cpp:2246-2441 recorded as alloc events
 * (csrc/hook.cpp:3364-3392); the reference never moves them, the build can. */
int fdy_archive_set_relocation(fdy_archive* a, const uint64_t* lo, const uint64_t* hi,
                               const uint64_t* new_lo, uint64_t n, uint32_t policy);

/* Use these template assignments instead of the key digests (the
 * graph_manifest.json path, csrc/CUDAGraphParallel.cpp:1735-1786).
 * template_of[i] == i marks a template.  Pass NULL to go back to digests. */
int fdy_archive_set_groups(fdy_archive* a, const uint32_t* template_of);

/* Template assignments from the text of a graph_manifest.json
 * (csrc/CUDAGraphParallel.cpp:1727-1786, written by python/foundry/graph.py:
 * 170-242).  names[i] is graph i's file name as the manifest lists it (the
 * ".json" name).  A group whose template is not among the names is skipped;
 * members not among the names are skipped; a later group overrides an
 * earlier one for the same member; a template's own entry is never set by
 * its group.  template_of[i] = i for templates and unlisted graphs.
 * If the text is not a manifest the reference accepts (not JSON, no
 * topology_groups array, a group without a string template or members
 * array), *used = 0 and template_of is untouched: the reference then groups
 * by keys.  A graph that ends up a member whose template is itself a member
 * (the reference builds no exec for such a template) is FDY_E_INVALID.
 * No device needed. */
int fdy_manifest_groups(const char* text, uint64_t len, const char* const* names, uint32_t n,
                        uint32_t* template_of, int* used);
/* fdy_manifest_groups, then fdy_archive_set_groups when the manifest is used
 * (otherwise the archive keeps grouping by keys). */
int fdy_archive_set_manifest(fdy_archive* a, const char* text, uint64_t len, const char* const* names,
                             int* used);

/* The GPU restore, enqueued on `stream`:
 *   1. digests per graph (CRC-64/XZ): saved topology key, dependency table,
 *      recomputed node-type stream, kernel-entry stream;
 *   2. template_of[g] = lowest index with an identical saved topology key
 *      (csrc/CUDAGraphParallel.cpp:1788-1851): found by a 64-bit word hash
 *      of the key and its length, then compared byte for byte (a hash or
 *      digest collision never merges two keys);
 *   3. per node: layout/descriptor compare against the template, param-image
 *      layout, memset/memcpy pointer relocation;
 *   4. fused diff + relocate over every param word: writes the relocated
 *      param image R_g of every graph and the override set O_g of every
 *      non-template graph in canonical (node, word) order.
 * Also resets every group's live image to its template. */
int fdy_restore(fdy_archive* a, void* stream);

/* Results.  Each synchronizes `stream`. */
int fdy_get_digests(fdy_archive* a, void* stream, uint64_t* out /* 4*G: key,edge,type,kent */);
int fdy_get_groups(fdy_archive* a, void* stream, uint32_t* template_of /* G */);
int fdy_get_graph_status(fdy_archive* a, void* stream, uint32_t* status /* G */);
int fdy_get_override_offsets(fdy_archive* a, void* stream, uint64_t* offsets /* G+1 */);
/* Param bytes per graph: sum of kernel param sizes (or extra arg-buffer
 * sizes) over nodes whose ranges are in bounds -- the bytes
 * prepare_on_demand_graph_binary copies (csrc/CUDAGraphParallel.cpp:1391-1409). */
int fdy_get_param_bytes(fdy_archive* a, void* stream, uint64_t* out /* G */);
int fdy_get_overrides(fdy_archive* a, void* stream, uint32_t graph, fdy_override* out, uint64_t cap,
                      uint64_t* n_out);
int fdy_get_node_flags(fdy_archive* a, void* stream, uint32_t graph, uint8_t* flags, uint64_t cap,
                       uint64_t* n_out);
int fdy_get_node_words(fdy_archive* a, void* stream, uint32_t graph, uint32_t* word_offsets /* N+1 */,
                       uint64_t cap, uint64_t* n_out);
/* The relocated param image R_g (node-major; each param padded to 8 B with zeros). */
int fdy_get_param_image(fdy_archive* a, void* stream, uint32_t graph, uint64_t* words, uint64_t cap,
                        uint64_t* n_out);
/* Relocated memset dst / memcpy dst,src per node (0 for other node types). */
int fdy_get_node_pointers(fdy_archive* a, void* stream, uint32_t graph, uint64_t* ptrs /* 2*N */,
                          uint64_t cap, uint64_t* n_out);

/* The bytes of one section (FDY_SEC_*, include/fdy_format.h) of graph
 * `graph`'s archive, e.g. the ALLOCATOR_EVENTS or OUTPUT_TENSORS JSON text
 * (csrc/CUDAGraphParallel.cpp:1664-1690 reads the same).  Works before
 * fdy_restore.  Synchronizes the device copy. */
int fdy_get_section(fdy_archive* a, uint32_t graph, uint32_t section, uint8_t* out, uint64_t cap, uint64_t* n_out);

/* Switch the live image of graph `graph`'s group to `graph`: restore the
 * template's words under the current graph's overrides that `graph` does
 * not override, write `graph`'s overrides, and point layout/descriptor-
 * changed nodes at `graph`.  Afterwards the live image equals R_graph on
 * every node without FDY_NODE_LAYOUT.  Counterpart of the all-node re-set
 * in csrc/CUDAGraph.cpp:340-461.  Enqueued on `stream`; no-op if current. */
int fdy_switch(fdy_archive* a, uint32_t graph, void* stream);

/* fdy_switch for each of targets[0..n) in order, enqueued on `stream`: the
 * same end state and the same scatter work per switch, with the checks and
 * the device selection done once for the whole sequence instead of per call
 * (for callers that switch graphs many times between launches, and for
 * measuring sustained switches).  Every group goes through its own switches
 * in sequence order; switches of different groups, which touch disjoint
 * state, share launches (unless a group graph holds one of the groups:
 * then the sequence's order is kept throughout).  Every target, and every
 * switch's launch size, is checked before any switch is enqueued: an
 * invalid target or a switch too large for one launch enqueues nothing.  A
 * HIP failure while enqueueing (or in a bound group graph's exec update)
 * returns at once: the switches already enqueued are recorded as their
 * groups' current graphs, none after them.  Counterpart of n calls of the
 * on-demand branch of csrc/CUDAGraph.cpp:330-461. */
int fdy_switch_sequence(fdy_archive* a, const uint32_t* targets, uint64_t n, void* stream);
/* Live state of the group whose template is `template_graph`.  Synchronizes.
 * node_src[n] = graph whose own image supplies node n (template unless the
 * node has a layout or descriptor difference). */
int fdy_get_live(fdy_archive* a, void* stream, uint32_t template_graph, uint64_t* words, uint64_t cap,
                 uint32_t* node_src, uint64_t node_cap, uint32_t* current_graph);

/* Standalone relocation of packed u64 words already in device memory
 * (in and out may alias).  The plan holds the interval search structure:
 * about 16 root lines of 64 B per interval (2M intervals: about 2 GB of device
 * memory), built once for many relocations, against about 2 per interval for
 * the index beside a restored archive.  The table is checked on the host and
 * the index built on the current device (only the table is uploaded);
 * returns when it is built. */
int fdy_reloc_plan_create(const uint64_t* lo, const uint64_t* hi, const uint64_t* new_lo, uint64_t n,
                          uint32_t policy, fdy_reloc_plan** out);
int fdy_reloc_plan_destroy(fdy_reloc_plan* p);
int fdy_relocate_words(const fdy_reloc_plan* p, const uint64_t* d_in, uint64_t* d_out, uint64_t n_words,
                       void* stream);
/* The plan's interval index: its 64-byte lines (the root lines first, then
 * the lines below them), copied to `lines` (room for cap of them) with their
 * count in *n_lines (lines may be null to ask for the count).  The index is
 * built on the device, one thread per root line.  No counterpart in the
 * reference; for inspecting a plan and checking the device build against
 * the host build of the same index. */
int fdy_reloc_plan_lines(const fdy_reloc_plan* p, void* lines, uint64_t cap, uint64_t* n_lines);

/* fdy_relocate_words without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (serving
 * loops and harnesses that forbid hipMalloc).  It takes the table of
 * fdy_reloc_plan_create (validated the same way) and relocates n_words
 * words at d_in into d_out (which may alias) exactly as a plan of that table
 * would, but builds the interval index on the host and keeps it in a static
 * device array of FDY_STATIC_INDEX_BYTES bytes that each GPU holds until the
 * process ends: no hipMalloc, hipFree or other device or pinned allocation.
 * An index larger than the array (past 65,536 intervals spread like the
 * relocation-heavy workload's: 64-byte lines, two root lines per interval
 * rounded down to a power of two, plus about a line per four intervals in
 * crowded ranges) is FDY_E_CAPACITY before anything is enqueued.  A table
 * that differs from the one the array holds has its index built on the
 * host, copied in `stream`'s order and waited for; a call with the same
 * table (the same policy and the same lo, hi and new_lo words, compared
 * exactly) reuses the index as it stands and only enqueues the relocation.
 * Every call on one GPU shares the array: calls on different streams that
 * overlap race (the later index can replace the earlier one under its
 * running kernel); calls in one stream's order do not. */
#define FDY_STATIC_INDEX_BYTES (8u << 20)
int fdy_relocate_words_static(const uint64_t* lo, const uint64_t* hi, const uint64_t* new_lo, uint64_t n,
                              uint32_t policy, const uint64_t* d_in, uint64_t* d_out, uint64_t n_words,
                              void* stream);

/* A non-owning DLPack view (a DLManagedTensor*, dlpack.h v0.8 layout) of
 * `ndim`-dimensional device memory at ptr: what the reference's output
 * tensors are (at::from_blob at the saved data_ptr, csrc/CUDAGraph.cpp:
 * 971-999), for a framework to import (torch.from_dlpack through a
 * "dltensor" capsule).  Its deleter frees only the view's own host block,
 * never the memory it describes.  NULL on bad arguments. */
void* fdy_dlpack_view(uint64_t ptr, int32_t device_type, int32_t device_id, int32_t ndim, const int64_t* shape,
                      const int64_t* strides, uint8_t code, uint8_t bits);

/* Timing of the last fdy_restore, from HIP events recorded on its stream
 * (milliseconds).  Synchronizes.  fdy_set_timing(a, 1) records an event
 * after every kernel; fdy_set_timing(a, 2) only at the start, between the
 * grouping + node passes and the diff phase, and at the end, so that no
 * event's wait for the kernel before it stretches a phase (the per-kernel
 * fields then read -1); 0 records none. */
typedef struct fdy_restore_timing {
  float group_ms;   /* key hashes and template assignment */
  float node_ms;    /* per-node compare, layout, and the four digests */
  float tmpl_ms;    /* relocation of the template graphs' param words */
  float diff_ms;    /* fused diff + relocate of every other graph's param words */
  float search_ms;  /* interval searches of the words left over by the diff; completed override records in place */
  float total_ms;
  float prepare_ms;     /* grouping and both node passes */
  float diff_phase_ms;  /* template, member and search passes */
} fdy_restore_timing;
int fdy_restore_timing_get(fdy_archive* a, fdy_restore_timing* out);
int fdy_set_timing(fdy_archive* a, int enabled);

/* How long the grouping step of fdy_restore waits for a lower graph's key
 * hash that its own workgroup has not yet published, in rounds of s_sleep
 * (about 64 ns each; default 16384, about 1 ms), before the waiting
 * workgroup hashes that key itself.  0 hashes every unpublished key at
 * once.  Results do not depend on it; it bounds how long one workgroup can
 * wait on another that is not resident.  No counterpart in the reference
 * (its grouping is a single-threaded map, csrc/CUDAGraphParallel.cpp:
 * 1788-1851). */
int fdy_set_group_wait(fdy_archive* a, uint32_t spins);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FOUNDRY_RESTORE_H */
