/*
 * foundry_region.h -- C ABI of the deterministic VMM allocation region and
 * its allocator-event record and replay, on HIP.
 *
 * The reference reserves one virtual-address region per process and serves
 * device allocations from a cursor inside it, so that SAVE and LOAD place
 * every allocation at the same address; LOAD replays the allocation events
 * each graph recorded and aborts if any address differs
 * (csrc/hook.cpp:3088-3142 set_allocation_region, 2246-2441 cuMemAlloc_v2,
 * 2626-2681 cuMemFree_v2, 2683-2773 cuMemAddressReserve, 3161-3298
 * preallocate_region, 3301-3352 current offset, 3354-3392 record/save,
 * 3394-3492 replay_hook_events_from_json).
 *
 * Here the same rules place allocations at the same OFFSETS from the region
 * base.  When the base the archive was saved with is free, the addresses are
 * the saved ones; when it is not (another mapping holds it), the region is
 * reserved elsewhere and fdy_region_intervals gives the interval table that
 * relocates every saved pointer (fdy_archive_set_relocation).
 *
 * Placement rules (identical to the reference's):
 *   alloc(bytes):   ptr = align_up(cursor, 2 MiB); mapped size = align_up(bytes, granularity);
 *                   cursor = align_up(ptr + bytes, 2 MiB)
 *   reserve(size, alignment), size < 2 GiB: ptr = align_up(cursor, alignment), nothing mapped;
 *                   cursor = align_up(ptr + size, 2 MiB)
 *   preallocate(size): one mapping of align_up(size, 2 MiB) at align_up(cursor, 2 MiB); later
 *                   allocations that start inside it are placed by the same rule without new
 *                   mappings, and must end inside it (else FDY_E_NOMEM)
 *
 * Conventions are those of foundry_restore.h.  A region is not safe for
 * concurrent use from several threads (the reference keeps it per thread).
 */
#ifndef FOUNDRY_REGION_H
#define FOUNDRY_REGION_H

#include <stddef.h>
#include <stdint.h>

#include "foundry_restore.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FDY_REGION_ALIGN (2ull << 20)     /* placement alignment of allocations */
#define FDY_REGION_SMALL_RESERVE (2ull << 30) /* reserves below this are carved from the region */

#define FDY_REGION_DEFAULT_BASE 0x200000000000ull /* the reference's is 0x500000000000 (csrc/hook.cpp:201) */

/* fdy_region_create flags */
#define FDY_REGION_EXACT_BASE 0x1u /* fail unless the region lies at `base` (the reference's rule) */

/* fdy_region_intervals modes */
#define FDY_REGION_IV_REGION 0u      /* one interval: [saved base, + size) -> actual base */
#define FDY_REGION_IV_ALLOCATIONS 1u /* one per allocation or reserve placed or replayed, sorted */

typedef struct fdy_region fdy_region;

typedef struct fdy_region_info {
  uint64_t saved_base;   /* the base asked for (the one the archive was saved with) */
  uint64_t base;         /* where the region is */
  uint64_t size;
  uint64_t offset;       /* cursor - base */
  uint64_t granularity;  /* mapping granularity of the device */
  uint64_t mapped_bytes; /* bytes of live mappings, preallocation included */
  uint64_t live_allocations;
  uint64_t prealloc_begin, prealloc_end; /* 0, 0 without a preallocation */
  uint64_t num_events;   /* recorded events */
  uint32_t recording;
  uint32_t flags;
} fdy_region_info;

/* Reserve the region (set_allocation_region).  `base` must be 2 MiB aligned;
 * `align` (a power of two >= 2 MiB, or 0 for 2 MiB) is the alignment asked
 * of the reservation when `base` is not free, and should be at least the
 * largest alignment the replayed reserves use.  The region is placed at
 * `base` only if the device can map memory there: on MI355X reservations at
 * or above 0x500000000000 (the reference's default base) are granted but
 * cannot be mapped, so such a base moves (or, with FDY_REGION_EXACT_BASE,
 * fails with FDY_E_STATE).  FDY_REGION_DEFAULT_BASE is mappable. */
int fdy_region_create(uint64_t base, uint64_t size, uint64_t align, uint32_t flags, fdy_region** out);
/* A planning region: the same placement arithmetic, events and replay, with
 * no device calls and nothing mapped.  It places allocations from `base` and
 * reads saved addresses relative to `saved_base` (both 2 MiB aligned);
 * `granularity` (0 = 2 MiB) only sizes the mappings it reports. */
int fdy_region_create_plan(uint64_t saved_base, uint64_t base, uint64_t size, uint64_t granularity,
                           fdy_region** out);
int fdy_region_destroy(fdy_region* r);
int fdy_region_info_get(fdy_region* r, fdy_region_info* out);

int fdy_region_alloc(fdy_region* r, uint64_t bytes, uint64_t* ptr);
/* Unknown pointers return FDY_E_RANGE (the reference hands them to the driver). */
int fdy_region_free(fdy_region* r, uint64_t ptr);
/* Carve a reservation (size < 2 GiB) from the region; nothing is mapped. */
int fdy_region_reserve(fdy_region* r, uint64_t size, uint64_t alignment, uint64_t* ptr);
int fdy_region_preallocate(fdy_region* r, uint64_t size);
int fdy_region_free_preallocated(fdy_region* r);
int fdy_region_get_offset(fdy_region* r, uint64_t* offset);
/* Move the cursor forward to base + offset (never backward: FDY_E_INVALID). */
int fdy_region_set_offset(fdy_region* r, uint64_t offset);

/* Event recording (start_hook_record / end_hook_record / clear_hook_events). */
int fdy_region_record(fdy_region* r, int enabled);
int fdy_region_clear_events(fdy_region* r);
/* The recorded events as the reference saves them in a graph's
 * ALLOCATOR_EVENTS section:
 *   {"start_base_addr":S,"events":[{"type":"alloc","size":N,"ptr":P},
 *    {"type":"free","ptr":P},{"type":"reserve","size":N,"ptr":P,"alignment":A}]}
 * *len receives the length; with buf == NULL or cap too small only *len is set
 * (FDY_E_CAPACITY in the second case). */
int fdy_region_events_json(fdy_region* r, char* buf, uint64_t cap, uint64_t* len);
/* Replay one graph's saved events (replay_hook_events_from_json): move the
 * cursor to the saved start, then place every alloc and reserve and undo
 * every free.  Saved addresses are read relative to the region's saved base;
 * any placement at another offset returns FDY_E_MISMATCH (the reference
 * aborts) and leaves the region as far as it got. */
int fdy_region_replay(fdy_region* r, const char* json, uint64_t len);
/* The relocation table from saved addresses to this region's
 * (FDY_REGION_IV_*).  n_out receives the count; with lo == NULL only the
 * count is returned. */
int fdy_region_intervals(fdy_region* r, uint32_t mode, uint64_t* lo, uint64_t* hi, uint64_t* new_lo, uint64_t cap,
                         uint64_t* n_out);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FOUNDRY_REGION_H */
