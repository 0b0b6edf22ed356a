// Parameter memory remap for the balloon path: the device memory of dropped
// weight layers becomes extend KV pages, and returns to the weights on
// restore (LlamaOp.pmm_drop / pmm_restore, called from
// kunserve/worker.py:454-501; the extend page ids num_base + k are
// kunserve/block_manager.py:262-269; the remap itself is described at
// kunserve/llm_engine.py:553-558).
//
// Built on HIP virtual memory. The K and V pools are each an address range
// reserved for base + max_extend pages, with one physical chunk backing the
// base pages. A weight segment is two physical chunks (its first and second
// half) mapped back to back at an address range of its own. Dropping a
// segment unmaps it there and maps its first half behind the K pool's last
// page and its second half behind the V pool's, so both pools grow in place:
// their addresses and every existing page id stay valid, and the new pages
// hold exactly the segment's bytes. Restoring undoes the most recent drop.
#include <vector>

#include "common.hpp"

struct kunserve_pmm {
  int device = 0;
  int64_t page_bytes = 0;
  int64_t base_pages = 0;
  int64_t max_pages = 0;    // base + max extend
  int64_t num_pages = 0;    // currently mapped, K and V alike
  char* k = nullptr;        // reserved ranges of max_pages * page_bytes
  char* v = nullptr;
  hipMemGenericAllocationHandle_t base_k = {}, base_v = {};
  bool has_base = false;
  struct Segment {
    int64_t bytes = 0;      // 2 * pages * page_bytes
    char* addr = nullptr;   // reserved range of `bytes`
    hipMemGenericAllocationHandle_t half[2] = {};
    bool home = false;      // mapped at addr
    bool dropped = false;   // mapped behind the pools
  };
  std::vector<Segment> segments;
  std::vector<int32_t> drop_order;   // stack of dropped segment ids
};

namespace kunserve {
namespace {

hipMemAllocationProp chunk_prop(int device) {
  hipMemAllocationProp prop = {};
  prop.type = hipMemAllocationTypePinned;
  prop.location.type = hipMemLocationTypeDevice;
  prop.location.id = device;
  return prop;
}

// Grants the device read/write access to [start, start + bytes), which
// must be mapped. Every grant starts at the beginning of its reservation and
// covers the whole mapped prefix: on a mapping that starts in the middle of
// a partly mapped reservation, hipMemSetAccess of just that mapping fails
// with an invalid-argument error in most runs (ROCm 7.2), while the prefix
// grant succeeds.
int grant(int device, char* start, int64_t bytes) {
  hipMemAccessDesc acc = {};
  acc.location.type = hipMemLocationTypeDevice;
  acc.location.id = device;
  acc.flags = hipMemAccessFlagsProtReadWrite;
  KSV_CHECK_HIP(hipMemSetAccess(start, size_t(bytes), &acc, 1));
  return KUNSERVE_OK;
}

// Maps both halves of a segment back to back from addr and grants access
// to the pair (all or nothing).
int map_pair(int device, char* addr, int64_t half, const hipMemGenericAllocationHandle_t* h) {
  KSV_CHECK_HIP(hipMemMap(addr, size_t(half), 0, h[0], 0));
  if (hipMemMap(addr + half, size_t(half), 0, h[1], 0) != hipSuccess) {
    (void)hipMemUnmap(addr, size_t(half));
    set_error("hipMemMap failed on the second half of a segment");
    return KUNSERVE_EHIP;
  }
  const int rc = grant(device, addr, 2 * half);
  if (rc != KUNSERVE_OK) {
    (void)hipMemUnmap(addr, size_t(half));
    (void)hipMemUnmap(addr + half, size_t(half));
  }
  return rc;
}

int64_t seg_pages(const kunserve_pmm* p, const kunserve_pmm::Segment& s) {
  return s.bytes / (2 * p->page_bytes);
}

// Unmaps and frees everything; each physical chunk is released once,
// wherever it is mapped at the time.
void release_all(kunserve_pmm* p) {
  (void)hipSetDevice(p->device);
  (void)hipDeviceSynchronize();
  while (!p->drop_order.empty()) {   // extend mappings, most recent first
    auto& s = p->segments[p->drop_order.back()];
    const int64_t n = seg_pages(p, s);
    const int64_t off = (p->num_pages - n) * p->page_bytes;
    (void)hipMemUnmap(p->k + off, size_t(n * p->page_bytes));
    (void)hipMemUnmap(p->v + off, size_t(n * p->page_bytes));
    p->num_pages -= n;
    s.dropped = false;
    p->drop_order.pop_back();
  }
  for (auto& s : p->segments) {
    const int64_t half = s.bytes / 2;
    if (s.home) {
      (void)hipMemUnmap(s.addr, size_t(half));
      (void)hipMemUnmap(s.addr + half, size_t(half));
    }
    for (auto h : s.half)
      if (h) (void)hipMemRelease(h);
    (void)hipMemAddressFree(s.addr, size_t(s.bytes));
  }
  p->segments.clear();
  if (p->has_base) {
    (void)hipMemUnmap(p->k, size_t(p->base_pages * p->page_bytes));
    (void)hipMemUnmap(p->v, size_t(p->base_pages * p->page_bytes));
  }
  if (p->base_k) (void)hipMemRelease(p->base_k);
  if (p->base_v) (void)hipMemRelease(p->base_v);
  if (p->k) (void)hipMemAddressFree(p->k, size_t(p->max_pages * p->page_bytes));
  if (p->v) (void)hipMemAddressFree(p->v, size_t(p->max_pages * p->page_bytes));
}

}  // namespace
}  // namespace kunserve

using namespace kunserve;

extern "C" int kunserve_pmm_create(int32_t device, int64_t page_bytes, int64_t base_pages,
                                   int64_t max_extend_pages, kunserve_pmm** out) {
  clear_error();
  KSV_CHECK_ARG(out, "null output");
  *out = nullptr;
  KSV_CHECK_ARG(page_bytes > 0 && base_pages > 0 && max_extend_pages >= 0,
                "bad page_bytes %lld / base_pages %lld / max_extend_pages %lld",
                (long long)page_bytes, (long long)base_pages, (long long)max_extend_pages);
  KSV_CHECK_ARG(base_pages + max_extend_pages < (int64_t(1) << 31), "too many pages");
  KSV_CHECK_HIP(hipSetDevice(device));
  int vmm = 0;
  KSV_CHECK_HIP(hipDeviceGetAttribute(&vmm, hipDeviceAttributeVirtualMemoryManagementSupported,
                                      device));
  if (!vmm) {
    set_error("device %d does not support virtual memory management", device);
    return KUNSERVE_EUNSUPPORTED;
  }
  hipMemAllocationProp prop = chunk_prop(device);
  size_t gran = 0;
  KSV_CHECK_HIP(hipMemGetAllocationGranularity(&gran, &prop, hipMemAllocationGranularityMinimum));
  KSV_CHECK_ARG(gran > 0 && page_bytes % int64_t(gran) == 0,
                "page_bytes %lld is not a multiple of the %zu-byte mapping granularity",
                (long long)page_bytes, gran);
  auto* p = new kunserve_pmm();
  p->device = device;
  p->page_bytes = page_bytes;
  p->base_pages = base_pages;
  p->max_pages = base_pages + max_extend_pages;
  const size_t reserve = size_t(p->max_pages * page_bytes);
  const size_t base = size_t(base_pages * page_bytes);
  int rc = KUNSERVE_EHIP;
  void* k = nullptr;
  void* v = nullptr;
  if (hipMemAddressReserve(&k, reserve, 0, nullptr, 0) != hipSuccess) k = nullptr;
  p->k = static_cast<char*>(k);
  if (p->k && hipMemAddressReserve(&v, reserve, 0, nullptr, 0) != hipSuccess) v = nullptr;
  p->v = static_cast<char*>(v);
  if (!p->k || !p->v) {
    set_error("cannot reserve 2 x %zu bytes of address space", reserve);
  } else if (hipMemCreate(&p->base_k, base, &prop, 0) != hipSuccess ||
             hipMemCreate(&p->base_v, base, &prop, 0) != hipSuccess) {
    set_error("out of device memory for 2 x %zu bytes of base pages", base);
  } else if (hipMemMap(p->k, base, 0, p->base_k, 0) != hipSuccess) {
    set_error("hipMemMap failed on the K base pages");
  } else if (hipMemMap(p->v, base, 0, p->base_v, 0) != hipSuccess) {
    (void)hipMemUnmap(p->k, base);
    set_error("hipMemMap failed on the V base pages");
  } else {
    p->has_base = true;
    if ((rc = grant(device, p->k, int64_t(base))) == KUNSERVE_OK &&
        (rc = grant(device, p->v, int64_t(base))) == KUNSERVE_OK) {
      p->num_pages = base_pages;
      *out = p;
      return KUNSERVE_OK;
    }
  }
  release_all(p);
  delete p;
  return rc;
}

extern "C" int kunserve_pmm_add_segment(kunserve_pmm* p, int64_t bytes, int32_t* segment_id,
                                        void** address) {
  clear_error();
  KSV_CHECK_ARG(p && segment_id && address, "null argument");
  KSV_CHECK_ARG(bytes > 0 && bytes % (2 * p->page_bytes) == 0,
                "segment bytes %lld must be a positive multiple of 2 x page_bytes (%lld)",
                (long long)bytes, (long long)(2 * p->page_bytes));
  KSV_CHECK_ARG(p->segments.size() < size_t(INT32_MAX), "too many segments");
  KSV_CHECK_HIP(hipSetDevice(p->device));
  kunserve_pmm::Segment s;
  s.bytes = bytes;
  const int64_t half = bytes / 2;
  void* addr = nullptr;
  KSV_CHECK_HIP(hipMemAddressReserve(&addr, size_t(bytes), 0, nullptr, 0));
  s.addr = static_cast<char*>(addr);
  hipMemAllocationProp prop = chunk_prop(p->device);
  int rc = KUNSERVE_EHIP;
  if (hipMemCreate(&s.half[0], size_t(half), &prop, 0) != hipSuccess ||
      hipMemCreate(&s.half[1], size_t(half), &prop, 0) != hipSuccess) {
    set_error("out of device memory for a %lld-byte segment", (long long)bytes);
  } else if ((rc = map_pair(p->device, s.addr, half, s.half)) == KUNSERVE_OK) {
    s.home = true;
    p->segments.push_back(s);
    *segment_id = int32_t(p->segments.size() - 1);
    *address = s.addr;
    return KUNSERVE_OK;
  }
  for (auto h : s.half)
    if (h) (void)hipMemRelease(h);
  (void)hipMemAddressFree(s.addr, size_t(bytes));
  return rc;
}

extern "C" int kunserve_pmm_drop(kunserve_pmm* p, int32_t segment_id, int64_t* num_pages) {
  clear_error();
  KSV_CHECK_ARG(p && num_pages, "null argument");
  KSV_CHECK_ARG(segment_id >= 0 && size_t(segment_id) < p->segments.size(),
                "segment %d does not exist", segment_id);
  auto& s = p->segments[segment_id];
  KSV_CHECK_ARG(!s.dropped, "segment %d is already dropped", segment_id);
  KSV_CHECK_ARG(s.home, "segment %d lost its mapping in a failed restore", segment_id);
  const int64_t n = seg_pages(p, s);
  const int64_t half = n * p->page_bytes;
  KSV_CHECK_ARG(p->num_pages + n <= p->max_pages,
                "dropping segment %d needs %lld extend pages, %lld left", segment_id,
                (long long)n, (long long)(p->max_pages - p->num_pages));
  KSV_CHECK_HIP(hipSetDevice(p->device));
  // Work already queued may still read the weights.
  KSV_CHECK_HIP(hipDeviceSynchronize());
  KSV_CHECK_HIP(hipMemUnmap(s.addr, size_t(half)));
  if (hipMemUnmap(s.addr + half, size_t(half)) != hipSuccess) {
    (void)hipMemMap(s.addr, size_t(half), 0, s.half[0], 0);
    (void)grant(p->device, s.addr, half);
    set_error("hipMemUnmap failed on segment %d", segment_id);
    return KUNSERVE_EHIP;
  }
  s.home = false;
  const int64_t off = p->num_pages * p->page_bytes;
  int rc = KUNSERVE_EHIP;
  if (hipMemMap(p->k + off, size_t(half), 0, s.half[0], 0) != hipSuccess) {
    set_error("hipMemMap failed behind the K pool");
  } else if (hipMemMap(p->v + off, size_t(half), 0, s.half[1], 0) != hipSuccess) {
    (void)hipMemUnmap(p->k + off, size_t(half));
    set_error("hipMemMap failed behind the V pool");
  } else if ((rc = grant(p->device, p->k, off + half)) != KUNSERVE_OK ||
             (rc = grant(p->device, p->v, off + half)) != KUNSERVE_OK) {
    (void)hipMemUnmap(p->k + off, size_t(half));
    (void)hipMemUnmap(p->v + off, size_t(half));
  }
  if (rc != KUNSERVE_OK) {
    // Put the segment back where it was and report the first failure.
    const std::string msg = kunserve_last_error();
    s.home = map_pair(p->device, s.addr, half, s.half) == KUNSERVE_OK;
    set_error("%s", msg.c_str());
    return rc;
  }
  s.dropped = true;
  p->num_pages += n;
  p->drop_order.push_back(segment_id);
  *num_pages = p->num_pages;
  return KUNSERVE_OK;
}

extern "C" int kunserve_pmm_restore(kunserve_pmm* p, int32_t* segment_id, int64_t* num_pages) {
  clear_error();
  KSV_CHECK_ARG(p && segment_id && num_pages, "null argument");
  KSV_CHECK_ARG(!p->drop_order.empty(), "no dropped segment to restore");
  const int32_t id = p->drop_order.back();
  auto& s = p->segments[id];
  const int64_t n = seg_pages(p, s);
  const int64_t half = n * p->page_bytes;
  KSV_CHECK_HIP(hipSetDevice(p->device));
  // Work already queued may still read the extend pages.
  KSV_CHECK_HIP(hipDeviceSynchronize());
  const int64_t off = (p->num_pages - n) * p->page_bytes;
  KSV_CHECK_HIP(hipMemUnmap(p->k + off, size_t(half)));
  if (hipMemUnmap(p->v + off, size_t(half)) != hipSuccess) {
    // Keep the pools whole: every page below num_pages stays mapped.
    if (hipMemMap(p->k + off, size_t(half), 0, s.half[0], 0) == hipSuccess)
      (void)grant(p->device, p->k, off + half);
    set_error("hipMemUnmap failed behind the V pool");
    return KUNSERVE_EHIP;
  }
  p->num_pages -= n;
  p->drop_order.pop_back();
  s.dropped = false;
  const int rc = map_pair(p->device, s.addr, half, s.half);
  s.home = rc == KUNSERVE_OK;
  if (rc != KUNSERVE_OK) return rc;
  *segment_id = id;
  *num_pages = p->num_pages;
  return KUNSERVE_OK;
}

extern "C" int kunserve_pmm_pools(const kunserve_pmm* p, void** k, void** v, int64_t* num_pages) {
  clear_error();
  KSV_CHECK_ARG(p && k && v && num_pages, "null argument");
  *k = p->k;
  *v = p->v;
  *num_pages = p->num_pages;
  return KUNSERVE_OK;
}

extern "C" void kunserve_pmm_destroy(kunserve_pmm* p) {
  if (!p) return;
  release_all(p);
  delete p;
}
