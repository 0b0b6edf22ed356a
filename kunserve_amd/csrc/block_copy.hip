// KV block movement for the paged pool: device block copy
// (LlamaOp.local_copy_blocks, kunserve/worker.py:818-823), kv_exchange pack
// and scatter (kunserve/flash_backend.py:930-985) and GPU<->host swap
// (torch.ops.swapping_ops.swap, kunserve/worker.py:646-650,673-681).
//
// Copy and pack/scatter are HBM-bound: every byte is read once and written
// once. One kernel serves all three: it walks "spans" (contiguous byte
// ranges) addressed through an optional id list on each side, and each
// workgroup streams a chunk of one span with 16-byte vector loads, eight
// loads in flight per lane before the first store.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace kunserve {
namespace {

// Two launch shapes: large spans (whole blocks of many layers) use
// 1024-thread workgroups that each stream 256 KiB (two rounds of 8 x 16 B
// per lane); slabs under 256 KiB use 256-thread workgroups on 32 KiB
// chunks. Both keep eight 16-byte loads per lane in flight before storing.
constexpr int kUnroll = 8;
constexpr int kSmallThreads = 256, kSmallRounds = 1;
constexpr int kLargeThreads = 1024, kLargeRounds = 2;
constexpr int64_t chunk_bytes(int threads, int rounds) { return int64_t(threads) * 16 * kUnroll * rounds; }

// One side of a copy: span s of item j lives at
//   base + id(j) * pitch + s * span_stride      (bytes)
// with id(j) = ids ? ids[j] : j. Items whose id is outside [0, limit) are
// skipped (the host validates ids; this only keeps a bad id from faulting).
struct Side {
  char* base;
  const int32_t* ids;
  int64_t pitch;
  int64_t span_stride;
  int64_t limit;
};

struct CopyJob {
  Side src;
  Side dst;
  int64_t n;             // items
  int32_t spans;         // spans per item
  int64_t span_bytes;    // multiple of 16
};

// Grid: x = item, y = chunk of the span, z = span. All index math is
// scalar; loads and stores are non-temporal (each byte is touched once).
template <int THREADS, int ROUNDS>
__global__ __launch_bounds__(THREADS) void span_copy_kernel(CopyJob job) {
  constexpr int64_t kChunk = chunk_bytes(THREADS, ROUNDS);
  constexpr int32_t kRound = THREADS * 16 * kUnroll;
  const int64_t item = blockIdx.x;
  const int64_t chunk = blockIdx.y;
  const int64_t span = blockIdx.z;

  const int64_t sid = job.src.ids ? job.src.ids[item] : item;
  const int64_t did = job.dst.ids ? job.dst.ids[item] : item;
  if (sid < 0 || sid >= job.src.limit || did < 0 || did >= job.dst.limit) return;

  const int64_t start = chunk * kChunk;
  const char* src = job.src.base + sid * job.src.pitch + span * job.src.span_stride + start;
  char* dst = job.dst.base + did * job.dst.pitch + span * job.dst.span_stride + start;
  const int32_t avail = int32_t(min<int64_t>(job.span_bytes - start, kChunk));
  const int32_t lane_off = int32_t(threadIdx.x) * 16;

  if (avail == kChunk) {
#pragma unroll 1
    for (int r = 0; r < ROUNDS; ++r) {
      u32x4 buf[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        buf[u] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(src + r * kRound + lane_off + u * THREADS * 16));
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        __builtin_nontemporal_store(
            buf[u], reinterpret_cast<u32x4*>(dst + r * kRound + lane_off + u * THREADS * 16));
    }
  } else {
    // Last, partial chunk of a span.
    for (int32_t off = lane_off; off < avail; off += THREADS * 16)
      *reinterpret_cast<u32x4*>(dst + off) = *reinterpret_cast<const u32x4*>(src + off);
  }
}

int launch_job(const CopyJob& job, hipStream_t stream) {
  if (job.n == 0 || job.spans == 0) return KUNSERVE_OK;
  const bool large = job.span_bytes >= chunk_bytes(kLargeThreads, kLargeRounds);
  const int64_t chunk = large ? chunk_bytes(kLargeThreads, kLargeRounds)
                              : chunk_bytes(kSmallThreads, kSmallRounds);
  const int64_t chunks = (job.span_bytes + chunk - 1) / chunk;
  KSV_CHECK_ARG(job.n < (int64_t(1) << 31), "copy of %lld items exceeds one launch",
                (long long)job.n);
  KSV_CHECK_ARG(chunks <= 65535 && job.spans <= 65535,
                "span of %lld bytes x %d spans exceeds the launch geometry",
                (long long)job.span_bytes, job.spans);
  dim3 grid(static_cast<unsigned>(job.n), static_cast<unsigned>(chunks),
            static_cast<unsigned>(job.spans));
  if (large)
    span_copy_kernel<kLargeThreads, kLargeRounds><<<grid, kLargeThreads, 0, stream>>>(job);
  else
    span_copy_kernel<kSmallThreads, kSmallRounds><<<grid, kSmallThreads, 0, stream>>>(job);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

int launch_jobs(const CopyJob& a, const CopyJob* b, hipStream_t stream) {
  int rc = launch_job(a, stream);
  if (rc || !b) return rc;
  return launch_job(*b, stream);
}

// Byte geometry of one page of one layer ("slab") in the pool.
struct SlabGeom {
  int64_t slab_bytes;     // num_kv_heads * page_size * head_dim * 2
  bool slab_dense;        // slab is one contiguous range
  bool block_dense;       // all layers of a page are one contiguous range
};

SlabGeom slab_geom(const kunserve_kv_pool* p) {
  SlabGeom g;
  const int64_t tok = p->head_dim;
  const int64_t head = int64_t(p->page_size) * tok;
  const int64_t slab = int64_t(p->num_kv_heads) * head;
  g.slab_bytes = slab * 2;
  g.slab_dense = p->token_stride == tok && (p->num_kv_heads == 1 || p->head_stride == head);
  g.block_dense = g.slab_dense && (p->num_layers == 1 || p->layer_stride == slab);
  return g;
}

}  // namespace
}  // namespace kunserve

using namespace kunserve;

extern "C" int kunserve_copy_blocks(const kunserve_kv_pool* pool, const int32_t* src_ids_dev,
                                    const int32_t* dst_ids_dev, int64_t n,
                                    kunserve_stream_t stream) {
  clear_error();
  int rc = check_pool(pool, false);
  if (rc) return rc;
  KSV_CHECK_ARG(n >= 0, "n < 0");
  if (n == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(src_ids_dev && dst_ids_dev, "null id array");
  const SlabGeom g = slab_geom(pool);
  KSV_CHECK_ARG(g.slab_dense, "copy_blocks needs dense [heads, page_size, head_dim] slabs");
  CopyJob job{};
  job.n = n;
  if (g.block_dense) {
    job.spans = 1;
    job.span_bytes = g.slab_bytes * pool->num_layers;
  } else {
    job.spans = pool->num_layers;
    job.span_bytes = g.slab_bytes;
  }
  for (Side* s : {&job.src, &job.dst}) {
    s->pitch = pool->page_stride * 2;
    s->span_stride = pool->layer_stride * 2;
    s->limit = pool->num_pages;
  }
  job.src.ids = src_ids_dev;
  job.dst.ids = dst_ids_dev;
  CopyJob jv = job;
  job.src.base = job.dst.base = static_cast<char*>(pool->k);
  jv.src.base = jv.dst.base = static_cast<char*>(pool->v);
  return launch_jobs(job, &jv, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int64_t kunserve_kv_pack_bytes(const kunserve_kv_pool* pool, int32_t num_layers,
                                          int64_t n) {
  if (!pool || num_layers < 0 || n < 0) return -1;
  return int64_t(num_layers) * n * 2 * slab_geom(pool).slab_bytes;
}

namespace {
// Pack (to_scratch) or scatter: pool pages <-> scratch
// [layers][n][K|V][num_kv_heads][page_size][head_dim].
int pack_or_scatter(const kunserve_kv_pool* pool, int32_t layer_begin, int32_t layer_end,
                    const int32_t* page_ids_dev, int64_t n, char* scratch,
                    int64_t scratch_bytes, bool to_scratch, hipStream_t stream) {
  clear_error();
  int rc = check_pool(pool, false);
  if (rc) return rc;
  KSV_CHECK_ARG(0 <= layer_begin && layer_begin <= layer_end && layer_end <= pool->num_layers,
                "layer range [%d, %d) outside [0, %d)", layer_begin, layer_end,
                pool->num_layers);
  KSV_CHECK_ARG(n >= 0, "n < 0");
  const int32_t nl = layer_end - layer_begin;
  if (n == 0 || nl == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(page_ids_dev && scratch, "null pointer");
  const SlabGeom g = slab_geom(pool);
  KSV_CHECK_ARG(g.slab_dense, "pack/scatter needs dense [heads, page_size, head_dim] slabs");
  const int64_t need = kunserve_kv_pack_bytes(pool, nl, n);
  if (scratch_bytes < need) {
    set_error("scratch holds %lld bytes, %lld needed", (long long)scratch_bytes,
              (long long)need);
    return KUNSERVE_ENOSPC;
  }
  CopyJob jobs[2];
  for (int kv = 0; kv < 2; ++kv) {
    CopyJob& job = jobs[kv];
    job = CopyJob{};
    job.n = n;
    job.spans = nl;
    job.span_bytes = g.slab_bytes;
    Side pool_side{};
    pool_side.base = static_cast<char*>(kv ? pool->v : pool->k) +
                     int64_t(layer_begin) * pool->layer_stride * 2;
    pool_side.ids = page_ids_dev;
    pool_side.pitch = pool->page_stride * 2;
    pool_side.span_stride = pool->layer_stride * 2;
    pool_side.limit = pool->num_pages;
    Side scr{};
    scr.base = scratch + kv * g.slab_bytes;
    scr.ids = nullptr;
    scr.pitch = 2 * g.slab_bytes;
    scr.span_stride = n * 2 * g.slab_bytes;
    scr.limit = n;
    job.src = to_scratch ? pool_side : scr;
    job.dst = to_scratch ? scr : pool_side;
  }
  return launch_jobs(jobs[0], &jobs[1], stream);
}
}  // namespace

extern "C" int kunserve_kv_pack(const kunserve_kv_pool* pool, int32_t layer_begin,
                                int32_t layer_end, const int32_t* page_ids_dev, int64_t n,
                                void* scratch_dev, int64_t scratch_bytes,
                                kunserve_stream_t stream) {
  return pack_or_scatter(pool, layer_begin, layer_end, page_ids_dev, n,
                         static_cast<char*>(scratch_dev), scratch_bytes, true,
                         reinterpret_cast<hipStream_t>(stream));
}

extern "C" int kunserve_kv_scatter(const kunserve_kv_pool* pool, int32_t layer_begin,
                                   int32_t layer_end, const int32_t* page_ids_dev, int64_t n,
                                   const void* scratch_dev, int64_t scratch_bytes,
                                   kunserve_stream_t stream) {
  return pack_or_scatter(pool, layer_begin, layer_end, page_ids_dev, n,
                         const_cast<char*>(static_cast<const char*>(scratch_dev)),
                         scratch_bytes, false, reinterpret_cast<hipStream_t>(stream));
}

namespace {
// Pinned host slots that hold a swap's (src, dst) id lists while its copy
// kernels read them. A slot is reused once the event recorded after its
// kernels has completed (hipEventQuery: no host wait); when every slot is
// still in flight a new one is allocated, up to kMaxSwapSlots, after which
// the oldest is waited for. Slots are per device and live until the
// process ends.
struct SwapIdSlot {
  int32_t* ids = nullptr;
  int64_t cap = 0;
  hipEvent_t done = nullptr;
  int device = -1;
  uint64_t used = 0;   // order of last use
  bool busy = false;   // handed out, event not yet recorded
};
constexpr size_t kMaxSwapSlots = 64;
// Ids a slot holds at least (src and dst of 8192 blocks, 64 KiB): slots
// are rarely regrown, and a regrowth frees a completed slot's buffer only.
constexpr int64_t kMinSwapSlotIds = 16384;
std::mutex g_swap_mu;
std::vector<SwapIdSlot> g_swap_slots;
uint64_t g_swap_clock = 0;

int acquire_swap_ids(int64_t count, hipStream_t s, int32_t** out) {
  int dev = 0;
  if (s)
    KSV_CHECK_HIP(hipStreamGetDevice(s, &dev));
  else
    KSV_CHECK_HIP(hipGetDevice(&dev));   // the null stream of the current device
  std::lock_guard<std::mutex> lock(g_swap_mu);
  SwapIdSlot* pick = nullptr;
  SwapIdSlot* oldest = nullptr;
  size_t on_dev = 0;
  for (SwapIdSlot& sl : g_swap_slots) {
    if (sl.device != dev || sl.busy) continue;
    ++on_dev;
    if (!oldest || sl.used < oldest->used) oldest = &sl;
    if (!pick && hipEventQuery(sl.done) == hipSuccess) pick = &sl;
  }
  (void)hipGetLastError();   // hipEventQuery reports hipErrorNotReady as an error
  if (!pick && on_dev >= kMaxSwapSlots && oldest) {
    KSV_CHECK_HIP(hipEventSynchronize(oldest->done));
    pick = oldest;
  }
  if (!pick) {
    int cur = 0;
    KSV_CHECK_HIP(hipGetDevice(&cur));
    if (cur != dev) KSV_CHECK_HIP(hipSetDevice(dev));
    SwapIdSlot sl;
    sl.device = dev;
    const hipError_t e = hipEventCreateWithFlags(&sl.done, hipEventDisableTiming);
    if (cur != dev) (void)hipSetDevice(cur);
    KSV_CHECK_HIP(e);
    g_swap_slots.push_back(sl);
    pick = &g_swap_slots.back();
  }
  if (pick->cap < count) {
    if (pick->ids) KSV_CHECK_HIP(hipHostFree(pick->ids));
    pick->ids = nullptr;
    pick->cap = 0;
    const int64_t cap = std::max<int64_t>(count, kMinSwapSlotIds);
    KSV_CHECK_HIP(hipHostMalloc(reinterpret_cast<void**>(&pick->ids), cap * sizeof(int32_t),
                                hipHostMallocDefault));
    pick->cap = cap;
  }
  pick->busy = true;
  pick->used = ++g_swap_clock;
  *out = pick->ids;
  return KUNSERVE_OK;
}

// Hands the slot holding `ids` back; when `launched`, it stays in use until
// the work now on stream s completes.
int release_swap_ids(int32_t* ids, hipStream_t s, bool launched) {
  std::lock_guard<std::mutex> lock(g_swap_mu);
  for (SwapIdSlot& sl : g_swap_slots) {
    if (sl.ids != ids) continue;
    sl.busy = false;
    if (launched) KSV_CHECK_HIP(hipEventRecord(sl.done, s));
    return KUNSERVE_OK;
  }
  set_error("swap id slot not found");
  return KUNSERVE_EINVAL;
}
}  // namespace

extern "C" int kunserve_swap_blocks(const int64_t* src_ids_host, const int64_t* dst_ids_host,
                                    int64_t n, int32_t is_swap_in, void* k_cache_dev,
                                    void* v_cache_dev, int64_t num_gpu_blocks,
                                    void* k_swap_host, void* v_swap_host,
                                    int64_t num_cpu_blocks, int64_t block_bytes,
                                    kunserve_stream_t stream) {
  clear_error();
  KSV_CHECK_ARG(n >= 0 && block_bytes > 0, "bad n or block_bytes");
  if (n == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(src_ids_host && dst_ids_host, "null id array");
  KSV_CHECK_ARG(k_cache_dev && v_cache_dev && k_swap_host && v_swap_host, "null pool pointer");
  const int64_t src_limit = is_swap_in ? num_cpu_blocks : num_gpu_blocks;
  const int64_t dst_limit = is_swap_in ? num_gpu_blocks : num_cpu_blocks;
  for (int64_t i = 0; i < n; ++i) {
    if (src_ids_host[i] < 0 || src_ids_host[i] >= src_limit || dst_ids_host[i] < 0 ||
        dst_ids_host[i] >= dst_limit) {
      set_error("swap pair %lld: %lld -> %lld outside [0, %lld) -> [0, %lld)", (long long)i,
                (long long)src_ids_host[i], (long long)dst_ids_host[i], (long long)src_limit,
                (long long)dst_limit);
      return KUNSERVE_ERANGE;
    }
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // The host pools are pinned: the copy kernel addresses them directly
  // (PCIe reads or writes from the CUs), one launch per pool for every
  // block, which keeps the host link busy; a copy call per block leaves it
  // idle between calls.
  void* k_host_dev = nullptr;
  void* v_host_dev = nullptr;
  const bool mapped = hipHostGetDevicePointer(&k_host_dev, k_swap_host, 0) == hipSuccess &&
                      hipHostGetDevicePointer(&v_host_dev, v_swap_host, 0) == hipSuccess &&
                      k_host_dev && v_host_dev;
  // The copy kernel takes block ids as int32.
  if (mapped && src_limit <= INT32_MAX && dst_limit <= INT32_MAX) {
    (void)hipGetLastError();
    int32_t* ids = nullptr;
    int rc = acquire_swap_ids(2 * n, s, &ids);
    if (rc) return rc;
    for (int64_t t = 0; t < n; ++t) {
      ids[t] = int32_t(src_ids_host[t]);
      ids[n + t] = int32_t(dst_ids_host[t]);
    }
    char* srcs[2] = {static_cast<char*>(is_swap_in ? k_host_dev : k_cache_dev),
                     static_cast<char*>(is_swap_in ? v_host_dev : v_cache_dev)};
    char* dsts[2] = {static_cast<char*>(is_swap_in ? k_cache_dev : k_host_dev),
                     static_cast<char*>(is_swap_in ? v_cache_dev : v_host_dev)};
    CopyJob jobs[2];
    for (int kv = 0; kv < 2; ++kv) {
      CopyJob& job = jobs[kv];
      job = CopyJob{};
      job.src = {srcs[kv], ids, block_bytes, 0, src_limit};
      job.dst = {dsts[kv], ids + n, block_bytes, 0, dst_limit};
      job.n = n;
      job.spans = 1;
      job.span_bytes = block_bytes;
    }
    rc = launch_jobs(jobs[0], &jobs[1], s);
    const int rr = release_swap_ids(ids, s, rc == KUNSERVE_OK);
    return rc ? rc : rr;
  }
  (void)hipGetLastError();
  // Host memory the device cannot address: one DMA copy per run of
  // consecutive ids.
  char* srcs[2] = {static_cast<char*>(is_swap_in ? k_swap_host : k_cache_dev),
                   static_cast<char*>(is_swap_in ? v_swap_host : v_cache_dev)};
  char* dsts[2] = {static_cast<char*>(is_swap_in ? k_cache_dev : k_swap_host),
                   static_cast<char*>(is_swap_in ? v_cache_dev : v_swap_host)};
  const hipMemcpyKind kind = is_swap_in ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
  int64_t i = 0;
  while (i < n) {
    int64_t j = i + 1;
    while (j < n && src_ids_host[j] == src_ids_host[j - 1] + 1 &&
           dst_ids_host[j] == dst_ids_host[j - 1] + 1)
      ++j;
    const int64_t bytes = (j - i) * block_bytes;
    for (int kv = 0; kv < 2; ++kv) {
      KSV_CHECK_HIP(hipMemcpyAsync(dsts[kv] + dst_ids_host[i] * block_bytes,
                                   srcs[kv] + src_ids_host[i] * block_bytes, bytes, kind, s));
    }
    i = j;
  }
  return KUNSERVE_OK;
}

// ------------------------------------------------- bandwidth calibration
// Flat streams with the launch shape of the large-span copy above (1024
// threads, 256 KiB per workgroup, eight 16-byte non-temporal accesses in
// flight per lane): reading only, writing only, and copying. They measure
// what this part's HBM gives each access mix, the ceiling the block copy is
// judged against.
namespace kunserve {
namespace {

constexpr int kProbeThreads = kLargeThreads;
constexpr int64_t kProbeChunk = chunk_bytes(kLargeThreads, kLargeRounds);

template <int MODE>   // 0 read, 1 write, 2 copy
__global__ __launch_bounds__(kProbeThreads) void hbm_probe_kernel(const char* src, char* dst) {
  constexpr int32_t kRound = kProbeThreads * 16 * kUnroll;
  const int64_t base = int64_t(blockIdx.x) * kProbeChunk + int32_t(threadIdx.x) * 16;
  u32x4 acc = {0u, 0u, 0u, 0u};
#pragma unroll 1
  for (int r = 0; r < kLargeRounds; ++r) {
    u32x4 buf[kUnroll];
    if constexpr (MODE != 1) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        buf[u] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(src + base + r * kRound + u * kProbeThreads * 16));
    } else {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        buf[u] = u32x4{uint32_t(base), uint32_t(r), uint32_t(u), 0x5a5a5a5au};
    }
    if constexpr (MODE == 0) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc ^= buf[u];
    } else {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        __builtin_nontemporal_store(
            buf[u], reinterpret_cast<u32x4*>(dst + base + r * kRound + u * kProbeThreads * 16));
    }
  }
  if constexpr (MODE == 0) {
    // Keeps the loads alive; the pattern cannot come from the caller's data
    // except by accident, and then only one 16-byte slot is written.
    if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0xf39cc060u &&
        acc[3] == 0x5851f42du)
      *reinterpret_cast<u32x4*>(dst) = acc;
  }
}

}  // namespace
}  // namespace kunserve

extern "C" int kunserve_hbm_probe(int32_t mode, const void* src_dev, void* dst_dev, int64_t bytes,
                                  kunserve_stream_t stream) {
  using namespace kunserve;
  clear_error();
  KSV_CHECK_ARG(mode >= 0 && mode <= 2, "mode %d is not 0 (read), 1 (write) or 2 (copy)", mode);
  KSV_CHECK_ARG(bytes > 0 && bytes % kProbeChunk == 0, "bytes must be a positive multiple of %lld",
                (long long)kProbeChunk);
  KSV_CHECK_ARG(dst_dev && aligned16(dst_dev) && (mode == 1 || (src_dev && aligned16(src_dev))),
                "null or misaligned buffer");
  const int64_t blocks = bytes / kProbeChunk;
  KSV_CHECK_ARG(blocks < (int64_t(1) << 31), "too many bytes for one launch");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const char* src = static_cast<const char*>(src_dev);
  char* dst = static_cast<char*>(dst_dev);
  const dim3 grid(static_cast<unsigned>(blocks));
  if (mode == 0)
    hbm_probe_kernel<0><<<grid, kProbeThreads, 0, s>>>(src, dst);
  else if (mode == 1)
    hbm_probe_kernel<1><<<grid, kProbeThreads, 0, s>>>(src, dst);
  else
    hbm_probe_kernel<2><<<grid, kProbeThreads, 0, s>>>(src, dst);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}
