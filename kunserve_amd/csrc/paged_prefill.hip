// Chunked-prefill attention with K/V append into pages (prefill rows of
// LlamaOp.pforward, kunserve/worker.py:298-312; chunk bounds
// kunserve/request.py:368-391,428-437; first index kunserve/request.py:447-462).
//
// Append: HBM-bound scatter of the new tokens' K/V rows into their pages.
//
// Attention: flash-attention style on fp16 MFMA (v_mfma_f32_32x32x16_f16,
// gfx950), fp32 accumulation and online softmax.
//  * Workgroup = 8 waves = 256 query rows of one (sequence, q head); each
//    wave owns 32 rows. Two waves share a SIMD, so one wave's softmax
//    (VALU, exp) overlaps the other's MFMAs.
//  * K/V tiles of 64 tokens are gathered from pages into double-buffered
//    LDS (K row-major, V transposed), both with XOR swizzles so that the
//    MFMA operand reads (ds_read_b128 for K, ds_read_b64 for V^T) and the
//    staging writes are free of bank conflicts. The next tile's global
//    loads are issued before the current tile's math, so their latency
//    hides behind it; one barrier per tile.
//  * S^T = K.Q^T is computed so that the accumulator layout (one query row
//    per lane column) is directly the B operand of O^T = V^T.P^T: the
//    probabilities never leave registers.
//  * Causal masking only on tiles that cross a wave's diagonal; tiles past
//    a wave's last visible position skip the math.
//  * The plan places the workgroups that read the same K/V (same sequence
//    and KV head) back to back on one XCD so that they share its L2.
#include <algorithm>
#include <vector>

#include "common.hpp"

namespace kunserve {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kTileQ = 32 * kWaves;   // query rows per workgroup (256)
constexpr int kTileKV = 64;           // kv tokens per iteration
constexpr int kD = 128;               // head_dim of the MFMA kernel
constexpr int kXcds = 8;              // MI355X: workgroup i runs on XCD i % 8
constexpr int kLoadsPerThread = kTileKV * kD / 8 / kThreads;   // 16-byte K (and V) loads

struct PrefillArgs {
  const f16* q;
  int64_t q_tok, q_head;
  f16* out;
  int64_t o_tok, o_head;
  const f16* k;   // pool K at the layer
  const f16* v;
  int64_t page_stride, head_stride, token_stride;
  int32_t num_pages;
  int32_t page_shift;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* kv_len;
  const int32_t* q_indptr;
  const int32_t* tiles;   // [num_tiles][3]: seq (-1: padding), first q row, q head
  int32_t ratio;
  float scale_log2;
};

// LDS layouts (element offsets within one buffer of kTileKV x kD halves;
// the two buffers differ in bit 13, so buffer selection is an XOR too).
// K: [token][dim], the 16-byte chunk index XORed with (token & 15).
//    offset(t, chunk) = (t*128 | (t & 15) << 3) ^ (chunk << 3)
__device__ __forceinline__ int sk_off(int t, int chunk) { return (t * kD | (t & 15) << 3) ^ (chunk << 3); }
// V^T: [dim][token], tokens of each row stored in MFMA k-slot order: chunk
// c = 2ks + h (8 halves) holds tokens 16ks + 4h + {0..3} and 16ks + 8 + 4h
// + {0..3}, so one ds_read_b128 is one A operand. Chunk index XORed with
// f(d) = (d ^ d >> 3) & 7.
//    offset(d, c) = (d*64 | f(d) << 3) ^ (c << 3)
__device__ __forceinline__ int vt_base(int d) { return d * kTileKV | ((d ^ (d >> 3)) & 7) << 3; }
__device__ __forceinline__ int vt_tok(int t) {   // (chunk << 3) | position of token t
  return ((2 * (t >> 4) + ((t >> 2) & 1)) << 3) | (((t >> 3) & 1) << 2) | (t & 3);
}
constexpr int kBufHalves = kTileKV * kD;   // 8192: bit 13

__global__ __launch_bounds__(kThreads) void paged_prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) f16 sK[2 * kBufHalves];
  __shared__ __attribute__((aligned(16))) f16 sV[2 * kBufHalves];

  const int32_t* item = a.tiles + 3 * blockIdx.x;
  const int seq = item[0];
  if (seq < 0) return;   // padding workgroup (uniform: no barrier reached)
  const int q0 = item[1];
  const int hq = item[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;       // query row within the wave / MFMA column
  const int h = lane >> 5;       // MFMA k-half

  const int hkv = hq / a.ratio;
  const int qb = a.q_indptr[seq];
  const int q_len = a.q_indptr[seq + 1] - qb;
  const int kvl = a.kv_len[seq];
  const int prefix = kvl - q_len;
  const int32_t* pages = a.indices + a.indptr[seq];
  const int page_mask = (1 << a.page_shift) - 1;

  const int qrow = q0 + wave * 32 + r;
  const bool row_ok = qrow < q_len;
  const int qpos = prefix + qrow;
  const bool wave_active = q0 + wave * 32 < q_len;
  const int wave_first_pos = prefix + q0 + wave * 32;
  const int wave_last_pos = prefix + min(q0 + wave * 32 + 31, q_len - 1);
  const int kv_end = prefix + min(q0 + kTileQ, q_len);   // exclusive
  const int ntiles = (kv_end + kTileKV - 1) / kTileKV;

  // Q as the B operand of S^T = K.Q^T: step s covers dims 16s + 8h .. +8.
  f16x8 qf[8];
  {
    const f16* qp = a.q + int64_t(qb + (row_ok ? qrow : 0)) * a.q_tok + int64_t(hq) * a.q_head;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = row_ok ? load_f16x8(qp + 16 * s + 8 * h) : f16x8{};
  }

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  float m = -1.0e30f;   // running max of this row, in scaled (log2) units
  float lsum = 0.f;     // this lane's share of the row sum (other half: lane ^ 32)

  const f16* kbase = a.k + int64_t(hkv) * a.head_stride;
  const f16* vbase = a.v + int64_t(hkv) * a.head_stride;

  f16x8 kr[kLoadsPerThread], vr[kLoadsPerThread];
  auto fetch = [&](int n0) {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      const int c = tid + kThreads * i;
      const int t = c >> 4, dc = c & 15;
      const int tok = n0 + t;
      const int p = tok < kvl ? pages[tok >> a.page_shift] : -1;
      if (p >= 0 && p < a.num_pages) {
        const int64_t off =
            int64_t(p) * a.page_stride + int64_t(tok & page_mask) * a.token_stride + dc * 8;
        kr[i] = load_f16x8(kbase + off);
        vr[i] = load_f16x8(vbase + off);
      } else {
        kr[i] = f16x8{};
        vr[i] = f16x8{};
      }
    }
  };
  auto stash = [&](int buf) {
    const int bo = buf * kBufHalves;
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      const int c = tid + kThreads * i;
      const int t = c >> 4, dc = c & 15;
      *reinterpret_cast<f16x8*>(&sK[bo ^ sk_off(t, dc)]) = kr[i];
      const int tv = vt_tok(t);
#pragma unroll
      for (int j = 0; j < 8; ++j) sV[bo ^ vt_base(dc * 8 + j) ^ tv] = vr[i][j];
    }
  };

  // Per-lane LDS bases (buffer 0); every operand address is one XOR away.
  const int kb0 = sk_off(r, h);            // K rows r (mt = 0) and r + 32 (^ 4096)
  int vb[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) vb[dt] = vt_base(32 * dt + r) ^ (h << 3);

  auto compute = [&](int buf, int n0) {
    const int bo = buf * kBufHalves;
    // S^T tiles: rows = kv tokens 32*mt + i, columns = query rows.
    f32x16 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int kb = bo ^ kb0 ^ (mt << 12);
      st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          *reinterpret_cast<const f16x8*>(&sK[kb]), qf[0], f32x16{}, 0, 0, 0);
#pragma unroll
      for (int s = 1; s < 8; ++s) {
        const f16x8 ka = *reinterpret_cast<const f16x8*>(&sK[kb ^ (s << 4)]);
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[s], st[mt], 0, 0, 0);
      }
    }
    // Lane holds tokens n0 + 32mt + 8(v/4) + 4h + v%4 of query row r.
    float mx = -INFINITY;
    if (n0 + kTileKV - 1 > wave_first_pos || n0 + kTileKV > kvl) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int tok = n0 + 32 * mt + 8 * (v >> 2) + 4 * h + (v & 3);
          if (tok > qpos || tok >= kvl) st[mt][v] = -INFINITY;
          mx = fmaxf(mx, st[mt][v]);
        }
    } else {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, st[mt][v]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * a.scale_log2;
    // Lazy running max: move it only when the tile's max exceeds it by more
    // than 8 (log2 units). Probabilities then stay <= 2^8 (exact in fp16 and
    // fp32), and the O rescale is skipped unless some row of the wave moved.
    if (__any(mx > m + 8.f)) {
      const float m_new = mx > m + 8.f ? mx : m;
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
    }

    // P^T as B operands: k-step ks covers tokens 16ks + 4h + {0..3} and
    // 16ks + 8 + 4h + {0..3}, i.e. accumulator entries v = 8(ks%2) + e of tile ks/2.
    f16x8 pb[4];
    float ps = 0.f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = fast_exp2(fmaf(st[mt][v], a.scale_log2, -m));
        ps += p;
        pb[2 * mt + (v >> 3)][v & 7] = f16(p);
      }
    lsum += ps;

    // O^T[dims, rows] += V^T[dims, tokens] . P^T[tokens, rows]
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const f16x8 va = *reinterpret_cast<const f16x8*>(&sV[bo ^ vb[dt] ^ (ks << 4)]);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[ks], o[dt], 0, 0, 0);
      }
    }
  };

  fetch(0);
  stash(0);
  __syncthreads();
  for (int it = 0; it < ntiles; ++it) {
    const int n0 = it * kTileKV;
    const int buf = it & 1;
    const bool more = it + 1 < ntiles;
    if (more) fetch(n0 + kTileKV);   // in flight during this tile's math
    if (wave_active && n0 <= wave_last_pos) compute(buf, n0);
    if (more) stash(buf ^ 1);        // that buffer was last read before the previous barrier
    __syncthreads();
  }

  lsum += __shfl_xor(lsum, 32);
  if (!row_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  f16* op = a.out + int64_t(qb + qrow) * a.o_tok + int64_t(hq) * a.o_head;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f16x4 val = {f16(o[dt][4 * g] * inv), f16(o[dt][4 * g + 1] * inv),
                         f16(o[dt][4 * g + 2] * inv), f16(o[dt][4 * g + 3] * inv)};
      *reinterpret_cast<f16x4*>(op + 32 * dt + 8 * g + 4 * h) = val;
    }
}

// ------------------------------------------------------------ append

struct AppendArgs {
  const f16* k_new;
  const f16* v_new;
  int64_t k_tok, k_head, v_tok, v_head;
  f16* k;   // pool at the layer
  f16* v;
  int64_t page_stride, head_stride, token_stride;
  int32_t num_pages;
  int32_t page_shift;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* kv_len;
  const int32_t* q_indptr;
  int32_t num_seqs;
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t chunks_per_row;   // head_dim / 8
};

__global__ __launch_bounds__(256) void append_kv_kernel(AppendArgs a) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_tok = int64_t(a.num_kv_heads) * a.chunks_per_row;
  if (idx >= int64_t(a.num_tokens) * per_tok) return;
  const int tok = int(idx / per_tok);
  if (tok >= a.q_indptr[a.num_seqs]) return;   // tokens not owned by any row
  const int rem = int(idx % per_tok);
  const int head = rem / a.chunks_per_row;
  const int dc = rem % a.chunks_per_row;
  // Row owning this token: largest b with q_indptr[b] <= tok.
  int lo = 0, hi = a.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.q_indptr[mid] <= tok) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int q_len = a.q_indptr[b + 1] - a.q_indptr[b];
  const int pos = a.kv_len[b] - q_len + (tok - a.q_indptr[b]);
  if (pos < 0 || pos >= a.kv_len[b]) return;
  const int p = a.indices[a.indptr[b] + (pos >> a.page_shift)];
  if (p < 0 || p >= a.num_pages) return;
  const int64_t dst = int64_t(p) * a.page_stride + int64_t(head) * a.head_stride +
                      int64_t(pos & ((1 << a.page_shift) - 1)) * a.token_stride + dc * 8;
  store_f16x8(a.k + dst, load_f16x8(a.k_new + int64_t(tok) * a.k_tok + int64_t(head) * a.k_head + dc * 8));
  store_f16x8(a.v + dst, load_f16x8(a.v_new + int64_t(tok) * a.v_tok + int64_t(head) * a.v_head + dc * 8));
}

}  // namespace
}  // namespace kunserve

using namespace kunserve;

extern "C" int kunserve_append_kv(const kunserve_kv_pool* pool, int32_t layer,
                                  const kunserve_page_table* table, const int32_t* q_indptr_dev,
                                  int32_t num_tokens, const kunserve_tensor3* k_new,
                                  const kunserve_tensor3* v_new, kunserve_stream_t stream) {
  clear_error();
  int rc = check_pool(pool, true);
  if (rc) return rc;
  KSV_CHECK_ARG(table && k_new && v_new, "null argument");
  KSV_CHECK_ARG(layer >= 0 && layer < pool->num_layers, "layer %d outside [0, %d)", layer,
                pool->num_layers);
  KSV_CHECK_ARG(num_tokens >= 0, "num_tokens < 0");
  if (num_tokens == 0 || table->num_seqs == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(q_indptr_dev && table->indptr_dev && table->indices_dev && table->kv_len_dev,
                "null table array");
  for (const kunserve_tensor3* t : {k_new, v_new})
    KSV_CHECK_ARG(t->data && aligned16(t->data) && t->token_stride % 8 == 0 &&
                      t->head_stride % 8 == 0,
                  "k_new / v_new must be 16-byte aligned with strides that are multiples of 8");
  AppendArgs a{};
  a.k_new = static_cast<const f16*>(k_new->data);
  a.v_new = static_cast<const f16*>(v_new->data);
  a.k_tok = k_new->token_stride;
  a.k_head = k_new->head_stride;
  a.v_tok = v_new->token_stride;
  a.v_head = v_new->head_stride;
  a.k = static_cast<f16*>(pool->k) + int64_t(layer) * pool->layer_stride;
  a.v = static_cast<f16*>(pool->v) + int64_t(layer) * pool->layer_stride;
  a.page_stride = pool->page_stride;
  a.head_stride = pool->head_stride;
  a.token_stride = pool->token_stride;
  a.num_pages = int32_t(pool->num_pages);
  a.page_shift = __builtin_ctz(pool->page_size);
  a.indptr = table->indptr_dev;
  a.indices = table->indices_dev;
  a.kv_len = table->kv_len_dev;
  a.q_indptr = q_indptr_dev;
  a.num_seqs = table->num_seqs;
  a.num_tokens = num_tokens;
  a.num_kv_heads = pool->num_kv_heads;
  a.chunks_per_row = pool->head_dim / 8;
  const int64_t threads = int64_t(num_tokens) * pool->num_kv_heads * a.chunks_per_row;
  const int64_t blocks = (threads + 255) / 256;
  KSV_CHECK_ARG(blocks < (int64_t(1) << 31), "append too large for one launch");
  append_kv_kernel<<<dim3(unsigned(blocks)), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(a);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

extern "C" int64_t kunserve_prefill_plan_bound(const int32_t* q_indptr_host, int32_t num_seqs,
                                               int32_t num_qo_heads) {
  if (num_seqs < 0 || num_qo_heads <= 0 || (num_seqs > 0 && !q_indptr_host)) return -1;
  int64_t tiles = 0;
  for (int32_t b = 0; b < num_seqs; ++b)
    tiles += (std::max(q_indptr_host[b + 1] - q_indptr_host[b], 0) + kTileQ - 1) / kTileQ;
  // Worst case: every item on one XCD, the others padded to the same depth.
  return 3 * kXcds * (tiles * num_qo_heads + 1);
}

extern "C" int kunserve_prefill_plan(const int32_t* q_indptr_host, const int32_t* kv_len_host,
                                     int32_t num_seqs, int32_t num_qo_heads,
                                     int32_t num_kv_heads, int32_t* plan_host,
                                     int64_t plan_capacity, kunserve_prefill_plan_info* info) {
  clear_error();
  KSV_CHECK_ARG(info && plan_host && num_seqs >= 0, "bad argument");
  KSV_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads, num_kv_heads);
  if (num_seqs > 0) KSV_CHECK_ARG(q_indptr_host && kv_len_host, "null q_indptr / kv_len");
  const int ratio = num_qo_heads / num_kv_heads;
  // A group = (sequence, KV head, q-tile range): its items (all `ratio` q
  // heads of each tile) read the same K/V. Groups go to XCDs greedily, most
  // work first. A (sequence, KV head) keeps all its tiles in one group
  // unless there are too few groups to spread over the XCDs.
  struct Group { int32_t seq, hkv, t0, t1; int64_t cost; };
  int64_t n_pairs = 0;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t ql = q_indptr_host[b + 1] - q_indptr_host[b];
    KSV_CHECK_ARG(ql >= 0, "q_indptr not monotone at %d", b);
    KSV_CHECK_ARG(kv_len_host[b] >= ql, "kv_len[%d] = %d < q_len %d", b, kv_len_host[b], ql);
    if (ql > 0) n_pairs += num_kv_heads;
  }
  const bool split_tiles = n_pairs < 2 * kXcds;
  std::vector<Group> groups;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t ql = q_indptr_host[b + 1] - q_indptr_host[b];
    if (ql == 0) continue;
    const int32_t prefix = kv_len_host[b] - ql;
    auto tile_cost = [&](int32_t q0) {
      return (int64_t(prefix) + std::min(q0 + kTileQ, ql)) * ratio;
    };
    for (int32_t g = 0; g < num_kv_heads; ++g) {
      if (split_tiles) {
        for (int32_t q0 = 0; q0 < ql; q0 += kTileQ)
          groups.push_back({b, g, q0, std::min(q0 + kTileQ, ql), tile_cost(q0)});
      } else {
        int64_t cost = 0;
        for (int32_t q0 = 0; q0 < ql; q0 += kTileQ) cost += tile_cost(q0);
        groups.push_back({b, g, 0, ql, cost});
      }
    }
  }
  std::stable_sort(groups.begin(), groups.end(),
                   [](const Group& x, const Group& y) { return x.cost > y.cost; });
  std::vector<std::vector<int32_t>> lanes(kXcds);
  int64_t load[kXcds] = {};
  for (const Group& g : groups) {
    const int x = int(std::min_element(load, load + kXcds) - load);
    load[x] += g.cost;
    for (int32_t q0 = g.t0; q0 < g.t1; q0 += kTileQ)
      for (int32_t hq = g.hkv * ratio; hq < (g.hkv + 1) * ratio; ++hq)
        lanes[x].insert(lanes[x].end(), {g.seq, q0, hq});
  }
  size_t depth = 0;
  for (const auto& l : lanes) depth = std::max(depth, l.size() / 3);
  const int64_t need = 3 * int64_t(depth) * kXcds;
  if (need > plan_capacity) {
    set_error("prefill plan needs %lld ints, capacity %lld", (long long)need,
              (long long)plan_capacity);
    return KUNSERVE_ENOSPC;
  }
  // Workgroup L runs on XCD L % 8: item i of XCD x goes to L = 8 i + x.
  for (size_t i = 0; i < depth; ++i)
    for (int x = 0; x < kXcds; ++x) {
      int32_t* dst = plan_host + 3 * (i * kXcds + x);
      if (3 * i < lanes[x].size()) {
        std::copy(lanes[x].begin() + 3 * i, lanes[x].begin() + 3 * i + 3, dst);
      } else {
        dst[0] = -1;
        dst[1] = dst[2] = 0;
      }
    }
  info->num_tiles = int32_t(depth * kXcds);
  info->tile_q = kTileQ;
  info->plan_ints = int32_t(need);
  info->num_qo_heads = num_qo_heads;
  return KUNSERVE_OK;
}

extern "C" int kunserve_paged_prefill(const kunserve_kv_pool* pool, int32_t layer,
                                      const kunserve_page_table* table,
                                      const int32_t* q_indptr_dev, const kunserve_tensor3* q,
                                      kunserve_tensor3* out, int32_t num_qo_heads,
                                      float sm_scale, const int32_t* plan_dev,
                                      const kunserve_prefill_plan_info* info,
                                      kunserve_stream_t stream) {
  clear_error();
  int rc = check_pool(pool, true);
  if (rc) return rc;
  KSV_CHECK_ARG(table && q && out && info, "null argument");
  KSV_CHECK_ARG(layer >= 0 && layer < pool->num_layers, "layer %d outside [0, %d)", layer,
                pool->num_layers);
  if (pool->head_dim != kD) {
    set_error("prefill kernel is compiled for head_dim %d, got %d", kD, pool->head_dim);
    return KUNSERVE_EUNSUPPORTED;
  }
  KSV_CHECK_ARG(num_qo_heads > 0 && num_qo_heads % pool->num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads,
                pool->num_kv_heads);
  KSV_CHECK_ARG(info->tile_q == kTileQ, "plan tile %d does not match kernel tile %d",
                info->tile_q, kTileQ);
  KSV_CHECK_ARG(info->num_qo_heads == num_qo_heads, "plan made for %d q heads, called with %d",
                info->num_qo_heads, num_qo_heads);
  if (info->num_tiles == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(plan_dev && q_indptr_dev && table->indptr_dev && table->indices_dev &&
                    table->kv_len_dev,
                "null plan or table array");
  KSV_CHECK_ARG(q->data && out->data && aligned16(q->data) && q->token_stride % 8 == 0 &&
                    q->head_stride % 8 == 0,
                "q must be 16-byte aligned with strides that are multiples of 8");
  KSV_CHECK_ARG((reinterpret_cast<uintptr_t>(out->data) & 7) == 0 && out->token_stride % 4 == 0 &&
                    out->head_stride % 4 == 0,
                "out must be 8-byte aligned with strides that are multiples of 4");
  PrefillArgs a{};
  a.q = static_cast<const f16*>(q->data);
  a.q_tok = q->token_stride;
  a.q_head = q->head_stride;
  a.out = static_cast<f16*>(out->data);
  a.o_tok = out->token_stride;
  a.o_head = out->head_stride;
  a.k = static_cast<const f16*>(pool->k) + int64_t(layer) * pool->layer_stride;
  a.v = static_cast<const f16*>(pool->v) + int64_t(layer) * pool->layer_stride;
  a.page_stride = pool->page_stride;
  a.head_stride = pool->head_stride;
  a.token_stride = pool->token_stride;
  a.num_pages = int32_t(pool->num_pages);
  a.page_shift = __builtin_ctz(pool->page_size);
  a.indptr = table->indptr_dev;
  a.indices = table->indices_dev;
  a.kv_len = table->kv_len_dev;
  a.q_indptr = q_indptr_dev;
  a.tiles = plan_dev;
  a.ratio = num_qo_heads / pool->num_kv_heads;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  paged_prefill_kernel<<<dim3(info->num_tiles), kThreads, 0,
                         reinterpret_cast<hipStream_t>(stream)>>>(a);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}
