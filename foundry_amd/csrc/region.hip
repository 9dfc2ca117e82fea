// region.hip -- host side of include/foundry_region.h: the deterministic VMM
// allocation region, its event record, and the replay that yields the
// relocation intervals.
//
// Every mapping gets a virtual-address reservation of its own, reserved at
// the address the placement rule gives (the hint must be honoured exactly).
// On MI355X with ROCm 7.2, hipMemSetAccess on a second mapping inside a
// shared reservation failed about two times in five, varying with the sizes
// and offsets of the other mappings, while every mapping alone in its
// reservation succeeded.  Creating a region checks that its range is free
// and that the device can map at its first and last pages.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/foundry_region.h"
#include "archive.h"
#include "json_min.h"

using fdy::err;

namespace {

constexpr uint64_t kAlign = FDY_REGION_ALIGN;

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) & ~(a - 1); }
bool pow2(uint64_t v) { return v && !(v & (v - 1)); }

std::string hex(uint64_t v) {
  char b[24];
  std::snprintf(b, sizeof b, "0x%llx", (unsigned long long)v);
  return b;
}

// One allocation, with its own mapping at `own_at` (its address) unless it
// lies inside the preallocation.
struct Mapping {
  uint64_t bytes = 0;     // requested
  uint64_t own_at = 0;
  uint64_t mapped = 0;    // bytes of the own mapping (0: wholly inside the preallocation)
  uint64_t reserved = 0;  // bytes of the own mapping's reservation (2 MiB multiple)
  hipMemGenericAllocationHandle_t handle{};
};

struct Event {
  enum Type { Alloc, Free, Reserve } type;
  uint64_t size = 0, ptr = 0, alignment = 0;
};

struct Interval {
  uint64_t lo, hi, new_lo;
};

}  // namespace

struct fdy_region {
  int device = 0;
  uint32_t flags = 0;
  uint64_t saved_base = 0, base = 0, size = 0, cursor = 0, granularity = kAlign;
  uint64_t pre_reserved = 0;  // bytes of the preallocation's reservation
  std::map<uint64_t, Mapping> maps;       // live allocations by address
  std::map<uint64_t, uint64_t> carved;    // reserves by address -> size
  bool has_pre = false;
  uint64_t pre_begin = 0, pre_end = 0;
  hipMemGenericAllocationHandle_t pre_handle{};
  bool recording = false;
  uint64_t record_start = 0;
  std::vector<Event> events;
  std::vector<Interval> placed;           // saved address range -> address here, in placement order

  bool plan = false;  // fdy_region_create_plan: arithmetic only
  bool dry() const { return plan; }

  ~fdy_region() {
    if (dry()) return;
    (void)hipSetDevice(device);
    for (auto& m : maps)
      if (m.second.mapped) {
        (void)hipMemUnmap(reinterpret_cast<void*>(m.second.own_at), m.second.mapped);
        (void)hipMemRelease(m.second.handle);
        (void)hipMemAddressFree(reinterpret_cast<void*>(m.second.own_at), m.second.reserved);
      }
    if (has_pre) {
      (void)hipMemUnmap(reinterpret_cast<void*>(pre_begin), pre_end - pre_begin);
      (void)hipMemRelease(pre_handle);
      (void)hipMemAddressFree(reinterpret_cast<void*>(pre_begin), pre_reserved);
    }
  }
};

namespace {

hipMemAllocationProp device_prop(int device) {
  hipMemAllocationProp p{};
  p.type = hipMemAllocationTypePinned;
  p.requestedHandleTypes = hipMemHandleTypeNone;
  p.location.type = hipMemLocationTypeDevice;
  p.location.id = device;
  return p;
}

// A reservation of `reserve` bytes exactly at `at` (a hint that is not
// honoured means another mapping holds part of the range), and physical
// memory of `bytes` (a granularity multiple) mapped read-write at its start.
int map_at(fdy_region* r, uint64_t at, uint64_t bytes, uint64_t reserve, hipMemGenericAllocationHandle_t* h) {
  void* p = nullptr;
  hipError_t e = hipMemAddressReserve(&p, reserve, kAlign, reinterpret_cast<void*>(at), 0);
  if (e != hipSuccess || reinterpret_cast<uint64_t>(p) != at) {
    (void)hipGetLastError();
    if (e == hipSuccess) (void)hipMemAddressFree(p, reserve);
    return err(FDY_E_STATE, "the range at " + hex(at) + " (" + std::to_string(reserve) +
                                " bytes) is held by another mapping");
  }
  const hipMemAllocationProp prop = device_prop(r->device);
  e = hipMemCreate(h, bytes, &prop, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // a failed call stays the last error until read
    (void)hipMemAddressFree(p, reserve);
    return err(FDY_E_NOMEM, "hipMemCreate of " + std::to_string(bytes) + " bytes failed: " + hipGetErrorString(e));
  }
  e = hipMemMap(p, bytes, 0, *h, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipMemRelease(*h);
    (void)hipMemAddressFree(p, reserve);
    return err(FDY_E_HIP, "hipMemMap at " + hex(at) + " of " + std::to_string(bytes) +
                              " bytes failed: " + hipGetErrorString(e));
  }
  hipMemAccessDesc acc{};
  acc.location.type = hipMemLocationTypeDevice;
  acc.location.id = r->device;
  acc.flags = hipMemAccessFlagsProtReadWrite;
  e = hipMemSetAccess(p, bytes, &acc, 1);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipMemUnmap(p, bytes);
    (void)hipMemRelease(*h);
    (void)hipMemAddressFree(p, reserve);
    return err(FDY_E_HIP, "hipMemSetAccess at " + hex(at) + " failed: " + hipGetErrorString(e));
  }
  return FDY_OK;
}

// Whether the device can map memory at `at` (2 MiB aligned, free): a
// reservation can be granted at an address the device cannot map (on
// MI355X, hints at or above 0x500000000000 are granted but refuse access),
// so one granularity page is mapped there in a reservation of its own,
// given access, and released.
bool device_can_map(fdy_region* r, uint64_t at) {
  hipMemGenericAllocationHandle_t h{};
  if (map_at(r, at, r->granularity, kAlign, &h) != FDY_OK) {
    fdy::g_err.clear();
    return false;
  }
  (void)hipMemUnmap(reinterpret_cast<void*>(at), r->granularity);
  (void)hipMemRelease(h);
  (void)hipMemAddressFree(reinterpret_cast<void*>(at), kAlign);
  return true;
}

void record(fdy_region* r, Event::Type t, uint64_t size, uint64_t ptr, uint64_t alignment) {
  if (r->recording) r->events.push_back(Event{t, size, ptr, alignment});
}

// Placement of `bytes` at the cursor (the cuMemAlloc_v2 rule, csrc/hook.cpp:2272-2291, 2424).
int place_alloc(fdy_region* r, uint64_t bytes, uint64_t* out) {
  if (bytes == 0) return err(FDY_E_INVALID, "zero-byte allocation");
  const uint64_t mapped = align_up(bytes, r->granularity);
  const uint64_t at = align_up(r->cursor, kAlign);
  if (at < r->base || at + mapped > r->base + r->size || at + mapped < at)
    return err(FDY_E_NOMEM, "region full: " + std::to_string(bytes) + " bytes at offset " + hex(at - r->base) +
                                " of a " + std::to_string(r->size) + "-byte region");
  Mapping m;
  m.bytes = bytes;
  m.own_at = at;
  if (r->has_pre && at >= r->pre_begin && at < r->pre_end) {
    // The fast path (csrc/hook.cpp:2279-2308): inside the preallocation, no
    // new mapping.  An allocation that would run past its end is refused: a
    // second mapping for the tail would make one allocation two memory
    // objects, which HIP copies refuse to span (the reference maps over the
    // preallocation, fails, and falls back to an address outside the region).
    if (at + bytes > r->pre_end)
      return err(FDY_E_NOMEM, std::to_string(bytes) + " bytes at offset " + hex(at - r->base) +
                                  " do not fit in the rest of the preallocation (it ends at offset " +
                                  hex(r->pre_end - r->base) + ")");
    m.mapped = 0;
  } else {
    m.mapped = mapped;
  }
  if (m.mapped) {
    m.reserved = align_up(m.mapped, kAlign);
    if (!r->dry()) {
      int rc = map_at(r, m.own_at, m.mapped, m.reserved, &m.handle);
      if (rc) return rc;
    }
  }
  r->maps[at] = m;
  r->cursor = align_up(at + bytes, kAlign);
  r->placed.push_back(Interval{at - r->base + r->saved_base, at - r->base + r->saved_base + bytes, at});
  record(r, Event::Alloc, bytes, at, 0);
  *out = at;
  return FDY_OK;
}

int place_reserve(fdy_region* r, uint64_t size, uint64_t alignment, uint64_t* out) {
  if (size == 0 || !pow2(alignment)) return err(FDY_E_INVALID, "reserve needs a size and a power-of-two alignment");
  if (size >= FDY_REGION_SMALL_RESERVE)
    return err(FDY_E_UNSUPPORTED, "reservations of 2 GiB or more are not carved from the region");
  const uint64_t at = align_up(r->cursor, alignment);
  if (at + size > r->base + r->size || at + size < at)
    return err(FDY_E_NOMEM, "region full: reserve of " + std::to_string(size) + " bytes");
  r->carved[at] = size;
  r->cursor = align_up(at + size, kAlign);
  r->placed.push_back(Interval{at - r->base + r->saved_base, at - r->base + r->saved_base + size, at});
  *out = at;
  return FDY_OK;
}

int do_free(fdy_region* r, uint64_t ptr) {
  auto it = r->maps.find(ptr);
  if (it == r->maps.end()) return err(FDY_E_RANGE, "pointer " + hex(ptr) + " is not an allocation of the region");
  const Mapping& m = it->second;
  if (m.mapped && !r->dry()) {
    FDY_HIP(hipMemUnmap(reinterpret_cast<void*>(m.own_at), m.mapped));
    FDY_HIP(hipMemRelease(m.handle));
    FDY_HIP(hipMemAddressFree(reinterpret_cast<void*>(m.own_at), m.reserved));
  }
  r->maps.erase(it);
  record(r, Event::Free, 0, ptr, 0);
  return FDY_OK;
}

bool uint_member(const fdy::json::Value& o, const char* key, uint64_t* v) {
  const fdy::json::Value* m = o.get(key);
  if (!m || m->kind != fdy::json::Value::Number || !m->is_uint) return false;
  *v = m->u;
  return true;
}

}  // namespace

extern "C" {

int fdy_region_create(uint64_t base, uint64_t size, uint64_t align, uint32_t flags, fdy_region** out) {
  if (!out) return err(FDY_E_INVALID, "null output pointer");
  *out = nullptr;
  if (align == 0) align = kAlign;
  if (!pow2(align) || align < kAlign) return err(FDY_E_INVALID, "alignment must be a power of two >= 2 MiB");
  if (base % kAlign) return err(FDY_E_INVALID, "region base " + hex(base) + " is not 2 MiB aligned");
  if (size == 0 || size % kAlign) return err(FDY_E_INVALID, "region size must be a nonzero multiple of 2 MiB");
  if (base + size < base) return err(FDY_E_INVALID, "region wraps the address space");
  auto r = std::make_unique<fdy_region>();
  r->flags = flags;
  r->saved_base = base;
  r->size = size;
  {
    FDY_HIP(hipGetDevice(&r->device));
    int vmm = 0;
    FDY_HIP(hipDeviceGetAttribute(&vmm, hipDeviceAttributeVirtualMemoryManagementSupported, r->device));
    if (!vmm) return err(FDY_E_UNSUPPORTED, "the device does not support virtual memory management");
    const hipMemAllocationProp prop = device_prop(r->device);
    size_t gran = 0;
    FDY_HIP(hipMemGetAllocationGranularity(&gran, &prop, hipMemAllocationGranularityMinimum));
    if (gran == 0 || kAlign % gran) return err(FDY_E_UNSUPPORTED, "mapping granularity does not divide 2 MiB");
    r->granularity = gran;
    // The range must be free (a hint at `base` honoured exactly) and the
    // device must be able to map at its first and last 2 MiB; otherwise the
    // region moves to a free range the device maps (or, with
    // FDY_REGION_EXACT_BASE, creation fails).  Nothing stays reserved: each
    // mapping reserves its own range when it is made.
    std::string why;
    auto range_ok = [&](uint64_t at) {
      void* p = nullptr;
      hipError_t e = hipMemAddressReserve(&p, size, align, reinterpret_cast<void*>(at), 0);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        why = std::string("reserving it failed: ") + hipGetErrorString(e);
        return false;
      }
      const uint64_t got = reinterpret_cast<uint64_t>(p);
      (void)hipMemAddressFree(p, size);
      if (got != at) {
        why = "part of it is taken (the reservation came back at " + hex(got) + ")";
        return false;
      }
      if (!device_can_map(r.get(), at)) {
        why = "the device cannot map its first page";
        return false;
      }
      if (!device_can_map(r.get(), at + size - kAlign)) {
        why = "the device cannot map its last page";
        return false;
      }
      return true;
    };
    uint64_t at = base;
    if (!range_ok(at)) {
      if (flags & FDY_REGION_EXACT_BASE)
        return err(FDY_E_STATE, "the range at " + hex(base) + " cannot hold the region: " + why);
      // hipMemAddressReserve does not always honour an alignment above 2 MiB:
      // reserve `align` more than needed and take the aligned address inside.
      void* p = nullptr;
      FDY_HIP(hipMemAddressReserve(&p, size + align, kAlign, nullptr, 0));
      at = align_up(reinterpret_cast<uint64_t>(p), align);
      (void)hipMemAddressFree(p, size + align);
      if (!range_ok(at))
        return err(FDY_E_HIP, "the fresh range at " + hex(at) + " cannot hold the region: " + why);
    }
    r->base = at;
  }
  r->cursor = r->base;
  *out = r.release();
  return FDY_OK;
}

int fdy_region_create_plan(uint64_t saved_base, uint64_t base, uint64_t size, uint64_t granularity,
                           fdy_region** out) {
  if (!out) return err(FDY_E_INVALID, "null output pointer");
  *out = nullptr;
  if (saved_base % kAlign || base % kAlign) return err(FDY_E_INVALID, "bases must be 2 MiB aligned");
  if (size == 0 || size % kAlign) return err(FDY_E_INVALID, "region size must be a nonzero multiple of 2 MiB");
  if (base + size < base || saved_base + size < saved_base) return err(FDY_E_INVALID, "region wraps the address space");
  if (granularity == 0) granularity = kAlign;
  if (!pow2(granularity) || granularity > kAlign) return err(FDY_E_INVALID, "granularity must be a power of two <= 2 MiB");
  auto r = std::make_unique<fdy_region>();
  r->plan = true;
  r->saved_base = saved_base;
  r->base = base;
  r->size = size;
  r->granularity = granularity;
  r->cursor = base;
  *out = r.release();
  return FDY_OK;
}

int fdy_region_destroy(fdy_region* r) {
  delete r;
  return FDY_OK;
}

int fdy_region_info_get(fdy_region* r, fdy_region_info* o) {
  if (!r || !o) return err(FDY_E_INVALID, "need a region and an output pointer");
  std::memset(o, 0, sizeof *o);
  o->saved_base = r->saved_base;
  o->base = r->base;
  o->size = r->size;
  o->offset = r->cursor - r->base;
  o->granularity = r->granularity;
  for (const auto& m : r->maps) o->mapped_bytes += m.second.mapped;
  if (r->has_pre) o->mapped_bytes += r->pre_end - r->pre_begin;
  o->live_allocations = r->maps.size();
  o->prealloc_begin = r->has_pre ? r->pre_begin : 0;
  o->prealloc_end = r->has_pre ? r->pre_end : 0;
  o->num_events = r->events.size();
  o->recording = r->recording ? 1 : 0;
  o->flags = r->flags;
  return FDY_OK;
}

int fdy_region_alloc(fdy_region* r, uint64_t bytes, uint64_t* ptr) {
  if (!r || !ptr) return err(FDY_E_INVALID, "need a region and an output pointer");
  if (!r->dry()) FDY_HIP(hipSetDevice(r->device));
  return place_alloc(r, bytes, ptr);
}

int fdy_region_free(fdy_region* r, uint64_t ptr) {
  if (!r) return err(FDY_E_INVALID, "null region");
  if (!r->dry()) FDY_HIP(hipSetDevice(r->device));
  return do_free(r, ptr);
}

int fdy_region_reserve(fdy_region* r, uint64_t size, uint64_t alignment, uint64_t* ptr) {
  if (!r || !ptr) return err(FDY_E_INVALID, "need a region and an output pointer");
  int rc = place_reserve(r, size, alignment, ptr);
  if (!rc) record(r, Event::Reserve, size, *ptr, alignment);
  return rc;
}

int fdy_region_preallocate(fdy_region* r, uint64_t size) {
  if (!r) return err(FDY_E_INVALID, "null region");
  if (size == 0) return err(FDY_E_INVALID, "zero-byte preallocation");
  if (r->has_pre) {
    int rc = fdy_region_free_preallocated(r);
    if (rc) return rc;
  }
  const uint64_t bytes = align_up(size, kAlign);  // so that its end is a 2 MiB boundary
  const uint64_t at = align_up(r->cursor, kAlign);
  if (at + bytes > r->base + r->size || at + bytes < at)
    return err(FDY_E_NOMEM, "region has no room for a " + std::to_string(bytes) + "-byte preallocation");
  if (!r->dry()) {
    FDY_HIP(hipSetDevice(r->device));
    int rc = map_at(r, at, bytes, align_up(bytes, kAlign), &r->pre_handle);
    if (rc) return rc;
  }
  r->pre_reserved = align_up(bytes, kAlign);
  // The cursor stays: allocations consume the preallocation as they come
  // (csrc/hook.cpp:3292-3294).
  r->has_pre = true;
  r->pre_begin = at;
  r->pre_end = at + bytes;
  return FDY_OK;
}

int fdy_region_free_preallocated(fdy_region* r) {
  if (!r) return err(FDY_E_INVALID, "null region");
  if (!r->has_pre) return FDY_OK;
  for (const auto& m : r->maps)
    if (m.first >= r->pre_begin && m.first < r->pre_end)
      return err(FDY_E_STATE, "allocation " + hex(m.first) + " still lives in the preallocation");
  if (!r->dry()) {
    FDY_HIP(hipSetDevice(r->device));
    FDY_HIP(hipMemUnmap(reinterpret_cast<void*>(r->pre_begin), r->pre_end - r->pre_begin));
    FDY_HIP(hipMemRelease(r->pre_handle));
    FDY_HIP(hipMemAddressFree(reinterpret_cast<void*>(r->pre_begin), r->pre_reserved));
  }
  r->has_pre = false;
  r->pre_begin = r->pre_end = 0;
  return FDY_OK;
}

int fdy_region_get_offset(fdy_region* r, uint64_t* offset) {
  if (!r || !offset) return err(FDY_E_INVALID, "need a region and an output pointer");
  *offset = r->cursor - r->base;
  return FDY_OK;
}

int fdy_region_set_offset(fdy_region* r, uint64_t offset) {
  if (!r) return err(FDY_E_INVALID, "null region");
  if (offset > r->size) return err(FDY_E_RANGE, "offset " + hex(offset) + " beyond the region");
  if (r->base + offset < r->cursor)
    return err(FDY_E_INVALID, "offset " + hex(offset) + " is behind the cursor " + hex(r->cursor - r->base) +
                                  " (the cursor never moves back)");
  r->cursor = r->base + offset;
  return FDY_OK;
}

int fdy_region_record(fdy_region* r, int enabled) {
  if (!r) return err(FDY_E_INVALID, "null region");
  if (enabled && !r->recording) r->record_start = r->cursor;
  r->recording = enabled != 0;
  return FDY_OK;
}

int fdy_region_clear_events(fdy_region* r) {
  if (!r) return err(FDY_E_INVALID, "null region");
  r->events.clear();
  return FDY_OK;
}

int fdy_region_events_json(fdy_region* r, char* buf, uint64_t cap, uint64_t* len) {
  if (!r || !len) return err(FDY_E_INVALID, "need a region and a length pointer");
  std::string s = "{\"start_base_addr\":" + std::to_string(r->record_start) + ",\"events\":[";
  for (size_t i = 0; i < r->events.size(); ++i) {
    const Event& e = r->events[i];
    if (i) s += ',';
    if (e.type == Event::Alloc)
      s += "{\"type\":\"alloc\",\"size\":" + std::to_string(e.size) + ",\"ptr\":" + std::to_string(e.ptr) + "}";
    else if (e.type == Event::Free)
      s += "{\"type\":\"free\",\"ptr\":" + std::to_string(e.ptr) + "}";
    else
      s += "{\"type\":\"reserve\",\"size\":" + std::to_string(e.size) + ",\"ptr\":" + std::to_string(e.ptr) +
           ",\"alignment\":" + std::to_string(e.alignment) + "}";
  }
  s += "]}";
  *len = s.size();
  if (!buf) return FDY_OK;
  if (cap < s.size()) return err(FDY_E_CAPACITY, "buffer holds " + std::to_string(cap) + " bytes, needs " +
                                                     std::to_string(s.size()));
  std::memcpy(buf, s.data(), s.size());
  return FDY_OK;
}

int fdy_region_replay(fdy_region* r, const char* text, uint64_t len) {
  if (!r || (!text && len)) return err(FDY_E_INVALID, "need a region and the events text");
  fdy::json::Value doc;
  std::string perr;
  fdy::json::Reader reader(text ? text : "", len);
  if (!reader.parse(doc, perr)) return err(FDY_E_FORMAT, "allocator events: " + perr);
  if (doc.kind != fdy::json::Value::Object) return err(FDY_E_FORMAT, "allocator events: not an object");
  if (!r->dry()) FDY_HIP(hipSetDevice(r->device));
  uint64_t start = 0;
  if (doc.get("start_base_addr")) {
    if (!uint_member(doc, "start_base_addr", &start)) return err(FDY_E_FORMAT, "start_base_addr is not an address");
    const uint64_t target = start - r->saved_base + r->base;
    if (start < r->saved_base || target < r->cursor)
      return err(FDY_E_MISMATCH, "the region's cursor is at offset " + hex(r->cursor - r->base) +
                                     " but the saved events start at offset " + hex(start - r->saved_base) +
                                     " (more was allocated before this graph than when it was saved)");
    if (target > r->base + r->size) return err(FDY_E_MISMATCH, "saved start lies beyond the region");
    r->cursor = target;
  }
  const fdy::json::Value* evs = doc.get("events");
  if (!evs || evs->kind != fdy::json::Value::Array) return err(FDY_E_FORMAT, "allocator events: no events array");
  for (size_t i = 0; i < evs->items.size(); ++i) {
    const fdy::json::Value& ev = evs->items[i];
    const fdy::json::Value* type = ev.kind == fdy::json::Value::Object ? ev.get("type") : nullptr;
    if (!type || type->kind != fdy::json::Value::String)
      return err(FDY_E_FORMAT, "allocator event " + std::to_string(i) + " has no type");
    uint64_t size = 0, ptr = 0, alignment = 0;
    if (!uint_member(ev, "ptr", &ptr)) return err(FDY_E_FORMAT, "allocator event " + std::to_string(i) + " has no ptr");
    const uint64_t want = ptr - r->saved_base;  // saved offset
    if (type->s == "alloc") {
      if (!uint_member(ev, "size", &size)) return err(FDY_E_FORMAT, "alloc event " + std::to_string(i) + " has no size");
      uint64_t got = 0;
      int rc = place_alloc(r, size, &got);
      if (rc) return rc;
      if (ptr < r->saved_base || got - r->base != want)
        return err(FDY_E_MISMATCH, "alloc event " + std::to_string(i) + " of " + std::to_string(size) +
                                       " bytes was saved at offset " + hex(want) + " but lands at offset " +
                                       hex(got - r->base));
    } else if (type->s == "reserve") {
      if (!uint_member(ev, "size", &size) || !uint_member(ev, "alignment", &alignment))
        return err(FDY_E_FORMAT, "reserve event " + std::to_string(i) + " lacks size or alignment");
      uint64_t got = 0;
      int rc = place_reserve(r, size, alignment, &got);
      if (rc) return rc;
      if (ptr < r->saved_base || got - r->base != want)
        return err(FDY_E_MISMATCH, "reserve event " + std::to_string(i) + " was saved at offset " + hex(want) +
                                       " but lands at offset " + hex(got - r->base) +
                                       " (is the region aligned as the reserve needs?)");
    } else if (type->s == "free") {
      // A free of an address the replay never placed is skipped, as the
      // reference reports and continues (csrc/hook.cpp:3481-3488).
      const uint64_t here = want + r->base;
      if (ptr >= r->saved_base && r->maps.count(here)) {
        int rc = do_free(r, here);
        if (rc) return rc;
      }
    } else {
      return err(FDY_E_FORMAT, "allocator event " + std::to_string(i) + " has unknown type '" + type->s + "'");
    }
  }
  return FDY_OK;
}

int fdy_region_intervals(fdy_region* r, uint32_t mode, uint64_t* lo, uint64_t* hi, uint64_t* new_lo, uint64_t cap,
                         uint64_t* n_out) {
  if (!r || !n_out) return err(FDY_E_INVALID, "need a region and a count pointer");
  std::vector<Interval> iv;
  if (mode == FDY_REGION_IV_REGION) {
    iv.push_back(Interval{r->saved_base, r->saved_base + r->size, r->base});
  } else if (mode == FDY_REGION_IV_ALLOCATIONS) {
    iv = r->placed;
    std::sort(iv.begin(), iv.end(), [](const Interval& a, const Interval& b) { return a.lo < b.lo; });
  } else {
    return err(FDY_E_INVALID, "unknown interval mode");
  }
  *n_out = iv.size();
  if (!lo) return FDY_OK;
  if (!hi || !new_lo) return err(FDY_E_INVALID, "need all three output arrays");
  if (cap < iv.size()) return err(FDY_E_CAPACITY, "arrays hold " + std::to_string(cap) + ", need " +
                                                      std::to_string(iv.size()));
  for (size_t i = 0; i < iv.size(); ++i) {
    lo[i] = iv[i].lo;
    hi[i] = iv[i].hi;
    new_lo[i] = iv[i].new_lo;
  }
  return FDY_OK;
}

}  // extern "C"
