/*
 * foundry_graph.h -- C ABI of the group graphs built from restored archives.
 *
 * A group graph is one hipGraph and one instantiated hipGraphExec per
 * topology group, built from the template's `.cugraph` nodes and dependency
 * table with the template's restored (relocated) param image.  Any graph of
 * the group is made runnable by fdy_group_graph_select: the device-side
 * override scatter (fdy_switch) moves the group's live param image to that
 * graph and mirrors every word it changes into host memory, and only the
 * nodes whose params or descriptor differ between the previous and the new
 * graph are re-set in the exec.
 *
 * Where the reference does this work (paths relative to the reference root):
 *   template graph from JSON      csrc/CUDAGraphParallel.cpp:171-834 (build_graph_from_parsed),
 *                                 run sequentially per template at 1944-1990
 *   shared exec per group         include/CUDAGraph.h:155-170 (SharedGraphExec),
 *                                 csrc/CUDAGraph.cpp:553-572 (link_on_demand_shared_exec)
 *   switch = re-set every node    csrc/CUDAGraph.cpp:330-461 (CUDAGraph::replay, on-demand branch)
 *   kernel identity               csrc/hook.cpp:315-321 (compute_hash: CRC-64/XZ of the module image),
 *                                 csrc/hook.cpp:3514-3551 (query_function_handle)
 *
 * Conventions are those of foundry_restore.h (int status, fdy_last_error,
 * streams passed as void*).  In addition:
 *   - A group graph keeps its archive alive in the sense that the archive
 *     refuses fdy_restore and fdy_archive_close until every group graph built
 *     on it is destroyed.  While a group graph exists, fdy_switch on its
 *     group behaves as fdy_group_graph_select.
 *   - Node kinds on gfx950: kernel nodes become kernel nodes; memset nodes
 *     become kernel nodes of the library's own fill kernel; memcpy nodes
 *     between device (or unified) memory become memcpy nodes; event record and
 *     wait nodes use one hipEvent per saved event id and group graph; empty
 *     nodes stay empty.  Dependencies name node ids (csrc/CUDAGraphParallel.cpp:774-800).
 *   - Launch attributes: cooperative is applied; cluster dimensions other
 *     than 1 are refused (gfx950 has no thread-block clusters); preferred
 *     cluster, scheduling policy, priority, memory-sync domain and shared
 *     memory carveout have no gfx950 counterpart and are not applied.
 */
#ifndef FOUNDRY_GRAPH_H
#define FOUNDRY_GRAPH_H

#include <stddef.h>
#include <stdint.h>

#include "foundry_restore.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fdy_registry fdy_registry;
typedef struct fdy_group_graph fdy_group_graph;

/* ---- code-object registry ------------------------------------------------
 * Code objects (gfx950 ELF images) are opaque bytes.  A code object's
 * identity is the CRC-64/XZ of its bytes, the `binary_hash` a kernel node of
 * a `.cugraph` names (csrc/hook.cpp:315-321); a kernel is (binary_hash, name)
 * (csrc/hook.cpp:3514-3551).  Loading happens on the device current at
 * fdy_registry_create. */
int fdy_registry_create(fdy_registry** out);
int fdy_registry_destroy(fdy_registry* r);
/* CRC-64/XZ of `size` bytes (no device needed). */
uint64_t fdy_code_object_hash(const void* bytes, uint64_t size);
/* Load a code object (hipModuleLoadData) and register it under its hash.
 * Adding bytes whose hash is already registered is a no-op. */
int fdy_registry_add(fdy_registry* r, const void* code_object, uint64_t size, uint64_t* binary_hash);
int fdy_registry_add_file(fdy_registry* r, const char* path, uint64_t* binary_hash);
/* hipFunction_t of kernel `name` in the code object `binary_hash`. */
int fdy_registry_lookup(fdy_registry* r, uint64_t binary_hash, const char* name, void** function);
/* Device address and size of the global variable `name` of the code object
 * `binary_hash` (hipModuleGetGlobal). */
int fdy_registry_global(fdy_registry* r, uint64_t binary_hash, const char* name, void** device_ptr,
                        uint64_t* bytes);

/* Kernel names of a code object (an ELF64 image, or an uncompressed clang
 * offload bundle holding one): the symbols with a kernel descriptor
 * (`name.kd`) in its symbol tables, sorted and '\n'-terminated, into buf
 * (*len = bytes needed; with buf NULL or cap below it, FDY_E_CAPACITY and
 * nothing written).  A malformed ELF image is FDY_E_FORMAT.  No device. */
int fdy_code_object_kernels(const void* code_object, uint64_t size, char* buf, uint64_t cap, uint64_t* len);

/* The packed code-object pair (csrc/hook.cpp:1589-1700, pack_fatbins_to_folder):
 * every code object registered in `r`, in registration order, into
 * dir/fatbin_image_packed.img as records {u64 binary_hash, u64 size, size
 * bytes} and dir/fatbin_entrypoint_packed.txt as, per record, the hash in 16
 * hex digits, the loader line "hipModuleLoadData,binary_flags=0", the number
 * of kernel names, the names (fdy_code_object_kernels), then "---".  gfx950
 * code objects are linked when built, so no record holds link segments.
 * `dir` is created if missing; *n_out = records written. */
int fdy_registry_pack(fdy_registry* r, const char* dir, uint32_t* n_out);
/* Load a pair written by fdy_registry_pack (csrc/hook.cpp:3787-3830): both
 * files must be present (FDY_E_IO otherwise); the two files must list the
 * same records, and every record's bytes must hash to its binary_hash and
 * name kernels its code object holds (FDY_E_FORMAT otherwise).  Each code
 * object is registered as fdy_registry_add does; *n_out = records read. */
int fdy_registry_load_packed(fdy_registry* r, const char* dir, uint32_t* n_out);

/* ---- group graphs ------------------------------------------------------- */
typedef struct fdy_group_graph_info {
  uint32_t template_graph;
  uint32_t current_graph;   /* graph whose params the exec holds */
  uint32_t num_nodes;
  uint32_t num_kernel_nodes;   /* kernel nodes of the archive */
  uint32_t num_fill_nodes;     /* memset nodes, run by the fill kernel */
  uint32_t num_memcpy_nodes;
  uint32_t num_event_nodes;
  uint32_t num_deps;
  uint32_t num_events;         /* distinct saved event ids */
  uint32_t num_execs;          /* execs instantiated (fdy_group_graph_set_exec_cache) */
  double build_ms;             /* host time of fdy_group_graph_create */
  double instantiate_ms;       /* of which hipGraphInstantiate */
} fdy_group_graph_info;

typedef struct fdy_select_stats {
  uint32_t nodes_reset;   /* nodes re-set in the exec */
  uint32_t kernel_nodes_reset;
  uint64_t words_scattered;  /* override records applied by the scatter(s) */
  double host_us;            /* wall time of the call, including the scatter's synchronization */
  double reset_us;           /* of which the exec node updates */
  double instantiate_us;     /* of which instantiating a new exec (0 unless the cache grew) */
  uint32_t cache_hit;        /* 1: an exec held the graph already; nothing was re-set or waited for */
  uint32_t pad_;
} fdy_select_stats;

/* Build the group graph of template graph `template_graph` after
 * fdy_restore: the group's live image goes back to the template, the nodes
 * are added in archive order with the template's relocated params, the
 * dependencies are added, and the graph is instantiated.  Synchronizes
 * `stream`.  Replaces the per-template JSON build
 * (csrc/CUDAGraphParallel.cpp:171-834, 1944-1990).
 *
 * The first group graph of an archive puts it in the serving layout: the
 * override records are packed to their count, live images are kept for
 * templates only, and the restore's scratch (candidates, ragged-word
 * sources) is freed; fdy_archive_info's device_bytes shows what is held.
 * fdy_restore, allowed again once the last group graph is destroyed,
 * allocates the scratch anew. */
int fdy_group_graph_create(fdy_archive* a, uint32_t template_graph, fdy_registry* r, void* stream,
                           fdy_group_graph** out);
int fdy_group_graph_destroy(fdy_group_graph* gg);
/* Make the group graph run graph `graph` (a member of the group).  A group
 * graph keeps up to max_execs instantiated execs (default 4), each holding
 * one graph's params.  If one holds `graph`, it becomes current: the
 * override scatter is enqueued on `stream` so that the group's live image
 * follows, and nothing else runs (no node update, no wait).  Otherwise the
 * least recently selected exec -- or a new one while there are fewer than
 * max_execs -- waits for its previous launch and takes `graph`'s params:
 * the scatter(s) on `stream` mark the nodes that differ between the two
 * graphs, then those nodes are re-set (after one synchronisation of
 * `stream`).  `stats` may be NULL.  Counterpart of the on-demand branch of
 * csrc/CUDAGraph.cpp:330-461, which has one exec per group and re-sets
 * every node on every switch. */
int fdy_group_graph_select(fdy_group_graph* gg, uint32_t graph, void* stream, fdy_select_stats* stats);
/* Re-set every node of the current exec from its graph, as the reference
 * does on every switch (csrc/CUDAGraph.cpp:345-441).  Use after an update
 * failed part-way; the bench uses it as the all-node baseline. */
int fdy_group_graph_reset_all(fdy_group_graph* gg, void* stream, fdy_select_stats* stats);
/* The number of execs the group graph keeps (at least 1; 1 is the
 * reference's one exec per group).  Lowering it destroys the least recently
 * selected execs past the limit (never the current one).  Each exec holds a
 * copy of every node's params (the driver's kernel-argument buffers). No
 * counterpart in the reference. */
int fdy_group_graph_set_exec_cache(fdy_group_graph* gg, uint32_t max_execs);
/* Launch the current exec on `stream` (csrc/CUDAGraph.cpp:476-477). */
int fdy_group_graph_launch(fdy_group_graph* gg, void* stream);
int fdy_group_graph_info_get(fdy_group_graph* gg, fdy_group_graph_info* out);
/* The group graph's hipGraph_t and its current hipGraphExec_t (either
 * pointer may be NULL), owned by the group graph: CUDAGraph::raw_cuda_graph
 * and raw_cuda_graph_exec (csrc/CUDAGraph.cpp:537-551) of every member.
 * The current exec changes with fdy_group_graph_select. */
int fdy_group_graph_handles(fdy_group_graph* gg, void** graph, void** exec);
/* hipGraphDebugDotPrint of the group graph, verbose, to `path`
 * (CUDAGraph::debug_dump, csrc/CUDAGraph.cpp:515-532). */
int fdy_group_graph_debug_dot(fdy_group_graph* gg, const char* path);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FOUNDRY_GRAPH_H */
