// Paged decode attention (q_len == 1 rows of LlamaOp.pforward,
// kunserve/worker.py:298-312; head counts kunserve/models.py:55-56, page
// size kunserve/models.py:57).
//
// HBM-bound: every K/V byte of a sequence is read exactly once per layer.
// Design for gfx950 (wave64, 256 CUs):
//  * The host plan cuts every sequence into partitions of part_tokens and
//    deals them, longest first, to 8 XCD lanes by estimated finish time;
//    the grid is lane entries x head groups, each XCD running all head
//    groups of one item at a time, so mixed context lengths still give an
//    even, device-filling grid that is dispatched longest item first on
//    every XCD.
//  * A workgroup (4 waves) owns one partition of one KV head and all
//    `G` query heads that share it (GQA: one KV read serves G heads).
//  * The partition's slice of the page table is staged in LDS once; after
//    that each K/V access is one 16-byte load per lane. A wave reads 1 KiB
//    of K and 1 KiB of V per load instruction (4 tokens x 256 B for
//    head_dim 128), four of each in flight per 16-token chunk.
//  * fp16 and bf16 pools (kernels are templates over the element type).
//  * Q.K uses v_dot2_f32_f16 / _bf16 and a DPP butterfly inside each 16-lane row;
//    the softmax is an online (running max) softmax in fp32 kept per row,
//    merged across rows with shuffles and across waves through LDS.
//  * Sequences longer than one partition write fp32 partial results with
//    their log-sum-exp (base 2); a small merge kernel combines them.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace kunserve {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kLoadsPerChunk = 4;        // 16-byte loads per lane per chunk (K and V each)
constexpr int kMaxPartTokens = 4096;
constexpr int kMinPageSize = 4;
constexpr int kMaxPartPages = kMaxPartTokens / kMinPageSize + 2;
constexpr int kMinPartTokens = 256;
constexpr int kXcds = 8;                 // MI355X: workgroup b runs on XCD b % 8
constexpr float kNegBig = -1.0e30f;      // finite "minus infinity" for running maxima

// Source of the loads of lanes past a partition's end and of bad page ids:
// one zero K/V row (head_dim <= 256), so loaded data is never masked.
__device__ __attribute__((aligned(16))) f16 g_zero_row[256];

struct DecodeArgs {
  const int32_t* q_token;   // null, or [num_seqs]: token of q and out of each sequence
  const f16* q;
  int64_t q_tok, q_head;
  f16* out;
  int64_t o_tok, o_head;
  const f16* k;             // pool K at the layer
  const f16* v;
  int64_t page_stride, head_stride, token_stride;
  int32_t num_pages;
  int32_t page_shift;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* work;      // [num_work][4]: seq (-1: padding), tok_begin, tok_end, slot (-1: direct)
  float* part_o;            // [slots][num_qo_heads][D]
  float* part_lse;          // [slots][num_qo_heads]
  int32_t num_qo_heads;
  int32_t head_groups;      // num_qo_heads / G
  int32_t num_work;         // work items of the plan
  int32_t ratio;            // num_qo_heads / num_kv_heads
  float scale_log2;         // sm_scale * log2(e)
};

// Work record and head group of workgroup b. The hardware hands workgroup
// b to XCD b % 8. The plan's records are 8 lanes interleaved (record
// 8 r + x is entry r of XCD x's lane), and XCD x runs every head group of
// its lane's entries in order, an entry's head groups back to back, so the
// pages an XCD reads at a time are those of its own few items (measured
// 1-2% faster than spreading each item's head groups over all XCDs). A
// lane's padding records (seq -1) end the workgroup at once.
__device__ __forceinline__ bool decode_work(const DecodeArgs& a, int& item, int& hg) {
  const int b = int(blockIdx.x);
  const int j = b >> 3;
  const int local = j / a.head_groups;
  hg = j - local * a.head_groups;
  item = 8 * local + (b & 7);
  return item < a.num_work;
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads) void paged_decode_kernel(DecodeArgs a) {
  typedef typename Vec<T>::v8 V8;
  constexpr int LPT = D / 8;            // lanes per token row (16 for D = 128)
  constexpr int TPL = kWave / LPT;      // tokens per load instruction (4)
  constexpr int CHUNK = TPL * kLoadsPerChunk;  // tokens per wave iteration (16)

  __shared__ int s_pages[kMaxPartPages];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];
  __shared__ float s_acc[kWaves][G][D];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int row = lane / LPT;
  const int col = lane % LPT;

  int item, hg;
  if (!decode_work(a, item, hg)) return;   // padding workgroup (uniform: no barrier reached)
  const int32_t* w = a.work + 4 * item;
  const int seq = w[0], tb = w[1], te = w[2], slot = w[3];
  if (seq < 0) return;   // a lane's padding record (uniform: no barrier reached)
  const int tok = a.q_token ? a.q_token[seq] : seq;   // q / out token of the sequence
  const int hq0 = hg * G;
  const int hkv = hq0 / a.ratio;
  const int page_mask = (1 << a.page_shift) - 1;

  // Stage this partition's page ids; invalid ids become -1 (masked).
  const int pb = tb >> a.page_shift;
  const int np = te > tb ? ((te - 1) >> a.page_shift) + 1 - pb : 0;
  const int32_t* seq_pages = a.indices + a.indptr[seq];
  for (int i = tid; i < np; i += kThreads) {
    const int p = seq_pages[pb + i];
    s_pages[i] = (p >= 0 && p < a.num_pages) ? p : -1;
  }

  V8 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qv[g] = load_v8<T>(a.q + int64_t(tok) * a.q_tok + int64_t(hq0 + g) * a.q_head + col * 8);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  }
  __syncthreads();

  const f16* kb = a.k + int64_t(hkv) * a.head_stride + col * 8;
  const f16* vb = a.v + int64_t(hkv) * a.head_stride + col * 8;
  const int nchunks = (te - tb + CHUNK - 1) / CHUNK;

  // One chunk = kLoadsPerChunk token rows per lane, K and V. Loads are
  // non-temporal: every K/V byte is read once, so it should not displace
  // the page table and q in the caches.
  struct Chunk {
    V8 k[kLoadsPerChunk], v[kLoadsPerChunk];
    bool ok[kLoadsPerChunk];
  };
  // Loads are issued unconditionally (lanes past the partition read the
  // cache-resident zero row): with no branch around them and no use of the
  // data until it is consumed, the compiler waits for the current chunk
  // while the next chunk's loads stay in flight.
  auto load_chunk = [&](int c, Chunk& ch) {
    const int t0 = tb + c * CHUNK;
#pragma unroll
    for (int i = 0; i < kLoadsPerChunk; ++i) {
      const int t = t0 + i * TPL + row;
      const int pi = min((t >> a.page_shift) - pb, kMaxPartPages - 1);
      const int p = (c < nchunks && t < te) ? s_pages[pi] : -1;
      ch.ok[i] = p >= 0;
      const int64_t off = int64_t(max(p, 0)) * a.page_stride + int64_t(t & page_mask) * a.token_stride;
      ch.k[i] = load_v8_nt<T>(ch.ok[i] ? kb + off : g_zero_row + col * 8);
      ch.v[i] = load_v8_nt<T>(ch.ok[i] ? vb + off : g_zero_row + col * 8);
    }
  };
  auto consume = [&](const Chunk& ch) {
    float vf[kLoadsPerChunk][8];
#pragma unroll
    for (int i = 0; i < kLoadsPerChunk; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) vf[i][j] = float(ch.v[i][j]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[kLoadsPerChunk];
      float mx = m[g];
#pragma unroll
      for (int i = 0; i < kLoadsPerChunk; ++i) {
        s[i] = group_sum<LPT>(dot8(qv[g], ch.k[i], 0.f)) * a.scale_log2;
        s[i] = ch.ok[i] ? s[i] : -INFINITY;
        mx = fmaxf(mx, s[i]);
      }
      const float alpha = fast_exp2(m[g] - mx);
      m[g] = mx;
      float p[kLoadsPerChunk];
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < kLoadsPerChunk; ++i) {
        p[i] = fast_exp2(s[i] - mx);
        ps += p[i];
      }
      l[g] = l[g] * alpha + ps;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = acc[g][j] * alpha;
#pragma unroll
        for (int i = 0; i < kLoadsPerChunk; ++i) x = fmaf(p[i], vf[i][j], x);
        acc[g][j] = x;
      }
    }
  };

  // Software pipeline over this wave's chunks (wave, wave + 4, ...): the
  // loads of the next chunk are in flight while the current one is reduced.
  if (wave < nchunks) {
    Chunk c0, c1;
    int c = wave;
    load_chunk(c, c0);
    while (true) {
      load_chunk(c + kWaves, c1);
      consume(c0);
      c += kWaves;
      if (c >= nchunks) break;
      load_chunk(c + kWaves, c0);
      consume(c1);
      c += kWaves;
      if (c >= nchunks) break;
    }
  }

  // Merge the TPL rows of each wave (lanes col, col+LPT, ...).
#pragma unroll
  for (int off = LPT; off < kWave; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m2 = __shfl_xor(m[g], off);
      const float l2 = __shfl_xor(l[g], off);
      const float mx = fmaxf(m[g], m2);
      const float f1 = fast_exp2(m[g] - mx), f2 = fast_exp2(m2 - mx);
      m[g] = mx;
      l[g] = l[g] * f1 + l2 * f2;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a2 = __shfl_xor(acc[g][j], off);
        acc[g][j] = acc[g][j] * f1 + a2 * f2;
      }
    }
  }
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (col == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s_acc[wave][g][col * 8 + j] = acc[g][j];
    }
  }
  __syncthreads();

  // Merge the waves and write the output (direct) or a partial (split).
  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int g = idx / D, d = idx % D;
    float mx = kNegBig;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) mx = fmaxf(mx, s_m[wv][g]);
    float lsum = 0.f, o = 0.f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) {
      const float f = fast_exp2(s_m[wv][g] - mx);
      lsum += s_l[wv][g] * f;
      o += s_acc[wv][g][d] * f;
    }
    const float r = lsum > 0.f ? o / lsum : 0.f;
    const int hq = hq0 + g;
    if (slot < 0) {
      reinterpret_cast<T*>(a.out)[int64_t(tok) * a.o_tok + int64_t(hq) * a.o_head + d] = T(r);
    } else {
      a.part_o[(int64_t(slot) * a.num_qo_heads + hq) * D + d] = r;
      if (d == 0)
        a.part_lse[int64_t(slot) * a.num_qo_heads + hq] =
            lsum > 0.f ? mx + __log2f(lsum) : -INFINITY;
    }
  }
}

// GQA decode on MFMA (head_dim 128, G = 8 query heads per KV head).
// With G query heads sharing each K/V byte the VALU form above needs ~G
// dot products and G x 8 FMAs per token row and lane, which caps it below
// the HBM rate for G = 8. Here both contractions run on
// v_mfma_f32_16x16x32_f16:
//  * K and V are read exactly as in the VALU kernel (each load instruction
//    covers 4 whole token rows, 1 KiB contiguous per wave: measured ~15%
//    more bandwidth than reading MFMA operands straight from memory) and
//    parked in a per-wave LDS block, row-major with the 16-byte chunk index
//    XORed with (token & 15).
//  * S^T[16 tokens x 16 heads] = K . Q^T, A operand = 16 K rows from LDS
//    (ds_read_b128), B operand = Q^T (head lane%16, zero for lanes >= G).
//  * O^T[16 dims x 16 heads] += V^T . P^T over 32 tokens: the A operand
//    gathers 8 tokens of one dim from the V rows (16-bit LDS reads, no
//    bank conflicts under the swizzle); P^T is the S^T accumulator itself
//    packed to fp16: lane (head j, group tg) holds tokens 4tg..4tg+3 of
//    each 16-token half, and the V gather uses the same token order.
//  * Online softmax per head column in fp32 with a lazy running max, merged
//    across waves through LDS; partial results as in the VALU kernel.
template <typename T, int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void paged_decode_mfma_kernel(DecodeArgs a) {
  typedef typename Vec<T>::v8 V8;
  constexpr int D = 128;
  constexpr int STEP = 32;                  // tokens per wave iteration
  constexpr int LOADS = STEP / 4;           // 16-byte loads per lane per step (K and V each)
  constexpr int BLK = STEP * D;             // halves per per-wave K (or V) block
  static_assert(G <= 16, "one 16-column MFMA tile of query heads");

  __shared__ int s_pages[kMaxPartPages];
  __shared__ int s_bad[kWaves];
  __shared__ __attribute__((aligned(16))) T s_kv[kWaves * BLK];   // 32 KiB: K, then V
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int j = lane & 15;     // MFMA row / column index of this lane
  const int tg = lane >> 4;    // MFMA k group / C row group
  const int lrow = lane >> 4;  // load layout: token row within a 4-row load
  const int lcol = lane & 15;  // load layout: 16-byte chunk of the row

  int item, hg;
  if (!decode_work(a, item, hg)) return;   // padding workgroup (uniform: no barrier reached)
  const int32_t* w = a.work + 4 * item;
  const int seq = w[0], tb = w[1], te = w[2], slot = w[3];
  if (seq < 0) return;   // a lane's padding record (uniform: no barrier reached)
  const int tok = a.q_token ? a.q_token[seq] : seq;   // q / out token of the sequence
  const int hq0 = hg * G;
  const int hkv = hq0 / a.ratio;
  const int page_mask = (1 << a.page_shift) - 1;

  const int pb = tb >> a.page_shift;
  const int np = te > tb ? ((te - 1) >> a.page_shift) + 1 - pb : 0;
  const int32_t* seq_pages = a.indices + a.indptr[seq];
  bool bad_id = false;
  for (int i = tid; i < np; i += kThreads) {
    const int p = seq_pages[pb + i];
    const bool ok = p >= 0 && p < a.num_pages;
    s_pages[i] = ok ? p : -1;
    bad_id |= !ok;
  }
  // Whether any staged id is outside the pool (one vote per wave, read after
  // the barrier below): only then do the scores need a per-page mask.
  const bool wave_bad = __any(bad_id);
  if (lane == 0) s_bad[wave] = wave_bad;

  // Q^T as the B operand: dim step s covers dims 32s + 8tg .. +8 of head j.
  V8 qb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qb[s] = j < G ? load_v8<T>(a.q + int64_t(tok) * a.q_tok + int64_t(hq0 + j) * a.q_head +
                               32 * s + 8 * tg)
                  : V8{};
  f32x4 o[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{};
  float m = kNegBig;   // running max of head j, scaled log2 units (same in all tg)
  float lsum = 0.f;    // this lane's share of head j's sum
  __syncthreads();
  int bad_votes = 0;
#pragma unroll
  for (int wv = 0; wv < kWaves; ++wv) bad_votes |= s_bad[wv];
  const bool any_bad = __builtin_amdgcn_readfirstlane(bad_votes) != 0;   // the same in every lane

  const f16* kb = a.k + int64_t(hkv) * a.head_stride + lcol * 8;
  const f16* vb = a.v + int64_t(hkv) * a.head_stride + lcol * 8;
  const int nsteps = (te - tb + STEP - 1) / STEP;
  T* sk = s_kv + wave * BLK;   // holds the step's K rows, then its V rows
  T* sv = sk;
  // Element (token t, dim d) of a block: t*128 + (((d >> 3) ^ (t & 15)) << 3) + (d & 7).
  auto blk_off = [](int t, int chunk) { return t * D + ((chunk ^ (t & 15)) << 3); };

  struct Step {
    V8 k[LOADS], v[LOADS];
  };
  // Unconditional loads (see the VALU kernel): past-the-end lanes and bad
  // page ids read the zero row.
  auto load_step = [&](int c, Step& st) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int t = tb + c * STEP + 4 * i + lrow;
      const int pi = min((t >> a.page_shift) - pb, kMaxPartPages - 1);
      const int p = (c < nsteps && t < te) ? s_pages[pi] : -1;
      const bool ok = p >= 0;
      const int64_t off = int64_t(max(p, 0)) * a.page_stride + int64_t(t & page_mask) * a.token_stride;
      st.k[i] = load_v8_nt<T>(ok ? kb + off : g_zero_row + lcol * 8);
      st.v[i] = load_v8_nt<T>(ok ? vb + off : g_zero_row + lcol * 8);
    }
  };
  auto stash = [&](const V8 (&rows)[LOADS]) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
      *reinterpret_cast<V8*>(&sk[blk_off(4 * i + lrow, lcol)]) = rows[i];
  };
  // Scores of the step whose K rows are in the block.
  auto scores = [&](f32x4 (&sc)[2]) {
    // LDS runs a wave's accesses in order; keep the compiler from moving them.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int t = 16 * sub + j;
      sc[sub] = f32x4{};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const V8 ka = *reinterpret_cast<const V8*>(&sk[blk_off(t, 4 * s + tg)]);
        sc[sub] = mfma16(ka, qb[s], sc[sub]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };
  // Softmax of the scores and O^T += V^T . P^T with the V rows in the block.
  auto accumulate = [&](f32x4 (&sc)[2], int c) {
    // Mask tokens past the partition; lane holds tokens 16 sub + 4 tg + v.
    // Tokens of an out-of-range page id (their K/V rows read as zeros) are
    // masked too, so they drop out of the softmax as in the VALU kernel; the
    // 4 tokens of a lane share one page (page_size >= 4).
    const int t0 = tb + c * STEP;
    float mx = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      bool bad_page = false;
      if (any_bad) {
        const int t = t0 + 16 * sub + 4 * tg;
        bad_page = t < te && s_pages[min((t >> a.page_shift) - pb, kMaxPartPages - 1)] < 0;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (bad_page || t0 + 16 * sub + 4 * tg + v >= te) sc[sub][v] = -INFINITY;
        mx = fmaxf(mx, sc[sub][v]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * a.scale_log2;
    if (__any(mx > m + 8.f)) {
      const float m_new = mx > m + 8.f ? mx : m;
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) o[mt] *= alpha;
    }
    V8 pb;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = fast_exp2(fmaf(sc[sub][v], a.scale_log2, -m));
        lsum += p;
        pb[sub * 4 + v] = T(p);
      }
    __builtin_amdgcn_wave_barrier();
    // O^T: A operand = V[token 16 sub + 4 tg + v][dim 16 mt + j] for e = 4 sub + v.
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const int d = 16 * mt + j;
      V8 va;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = 16 * (e >> 2) + 4 * tg + (e & 3);
        va[e] = sv[blk_off(t, d >> 3) + (d & 7)];
      }
      o[mt] = mfma16(va, pb, o[mt]);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // One register buffer: the next step's loads are issued once the current
  // step's K and V rows are parked in LDS, and land during its math.
  if (wave < nsteps) {
    Step st;
    int c = wave;
    load_step(c, st);
    while (c < nsteps) {
      f32x4 sc[2];
      stash(st.k);
      scores(sc);
      stash(st.v);   // overwrites the K rows: the score reads were issued first
      load_step(c + kWaves, st);
      accumulate(sc, c);
      c += kWaves;
    }
  }

  // Head j's sum over the 4 row groups of this wave.
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  __syncthreads();   // every wave is done with its K/V blocks: reuse them for the merge
  float* s_o = reinterpret_cast<float*>(s_kv);   // [kWaves][G][D]
  if (j < G) {
    if (tg == 0) {
      s_m[wave][j] = m;
      s_l[wave][j] = lsum;
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) s_o[(wave * G + j) * D + 16 * mt + 4 * tg + v] = o[mt][v];
  }
  __syncthreads();
  for (int idx = tid; idx < G * D; idx += kThreads) {
    const int g = idx / D, d = idx % D;
    float mxw = kNegBig;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) mxw = fmaxf(mxw, s_m[wv][g]);
    float ls = 0.f, acc = 0.f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) {
      const float f = fast_exp2(s_m[wv][g] - mxw);
      ls += s_l[wv][g] * f;
      acc += s_o[(wv * G + g) * D + d] * f;
    }
    const float r = ls > 0.f ? acc / ls : 0.f;
    const int hq = hq0 + g;
    if (slot < 0) {
      reinterpret_cast<T*>(a.out)[int64_t(tok) * a.o_tok + int64_t(hq) * a.o_head + d] = T(r);
    } else {
      a.part_o[(int64_t(slot) * a.num_qo_heads + hq) * D + d] = r;
      if (d == 0)
        a.part_lse[int64_t(slot) * a.num_qo_heads + hq] = ls > 0.f ? mxw + __log2f(ls) : -INFINITY;
    }
  }
}

// Combines the partitions of split sequences: one wave per (sequence,
// q head). Lane j first reads the log-sum-exp of partition j, so the
// weights come from one round of loads; each lane then accumulates D/64
// dimensions over the partitions.
template <typename T, int D>
__global__ __launch_bounds__(kWave) void decode_merge_kernel(const int32_t* merges,
                                                             const int32_t* q_token,
                                                             const float* part_o,
                                                             const float* part_lse, T* out,
                                                             int64_t o_tok, int64_t o_head,
                                                             int32_t num_qo_heads) {
  constexpr int DPL = D / kWave;
  typedef float PartVec __attribute__((ext_vector_type(DPL)));
  const int32_t* mg = merges + 4 * blockIdx.x;
  const int seq = mg[0], s0 = mg[1], n = mg[2];
  const int hq = blockIdx.y;
  const int lane = threadIdx.x;

  // Partials are read kBatch at a time, each batch's loads issued together
  // (one partial at a time waits a memory round trip per partial), and
  // summed in partition order, so the result does not depend on timing.
  // The first batch goes out with the first 64 log-sum-exps, before the
  // maximum they are weighted by is known.
  constexpr int kBatch = 8;
  PartVec x[kBatch];
  auto load_batch = [&](int first, int cnt) {   // partials first .. first + min(cnt, kBatch)
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const float* src = part_o + (int64_t(s0 + first + u) * num_qo_heads + hq) * D + lane * DPL;
      x[u] = u < cnt ? *reinterpret_cast<const PartVec*>(src) : PartVec{};
    }
  };
  float lse = lane < n ? part_lse[int64_t(s0 + lane) * num_qo_heads + hq] : -INFINITY;
  load_batch(0, n);
  float mx = lse;
  for (int j = lane + kWave; j < n; j += kWave)
    mx = fmaxf(mx, part_lse[int64_t(s0 + j) * num_qo_heads + hq]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));

  float o[DPL] = {};
  float wsum = 0.f;
  if (mx > -INFINITY) {
    for (int base = 0; base < n; base += kWave) {
      const int j = base + lane;
      if (base > 0) lse = j < n ? part_lse[int64_t(s0 + j) * num_qo_heads + hq] : -INFINITY;
      const float w = j < n ? fast_exp2(lse - mx) : 0.f;
      wsum += w;
      const int cnt = min(kWave, n - base);   // uniform
      for (int t0 = 0; t0 < cnt; t0 += kBatch) {
        if (base + t0 > 0) load_batch(base + t0, cnt - t0);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const float wt = __shfl(w, t0 + u);   // every lane: t0 + u < kWave
          if (t0 + u < cnt) {
#pragma unroll
            for (int e = 0; e < DPL; ++e) o[e] = fmaf(wt, x[u][e], o[e]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) wsum += __shfl_xor(wsum, off);
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int tok = q_token ? q_token[seq] : seq;
  T* dst = out + int64_t(tok) * o_tok + int64_t(hq) * o_head + lane * DPL;
#pragma unroll
  for (int e = 0; e < DPL; ++e) dst[e] = T(o[e] * inv);
}

int pick_group(int ratio) {
  for (int g : {8, 4, 2}) {
    if (ratio % g == 0) return g;
  }
  return 1;
}

template <typename T, int D>
int launch_decode(const DecodeArgs& a, int group, dim3 grid, hipStream_t s) {
  // Groups of 4 and 8 query heads per KV head run on MFMA (Llama-3-8B shape:
  // 6.05 TB/s vs 5.23 TB/s on VALU); for 1 and 2 the VALU kernel is as fast
  // (Llama-2-7B shape: 5.81 vs 5.78 TB/s) and leaves LDS idle.
  if constexpr (D == 128) {
    if (group == 4 || group == 8) {
      if (group == 4)
        paged_decode_mfma_kernel<T, 4><<<grid, kThreads, 0, s>>>(a);
      else
        paged_decode_mfma_kernel<T, 8><<<grid, kThreads, 0, s>>>(a);
      KSV_CHECK_LAUNCH();
      return KUNSERVE_OK;
    }
  }
  switch (group) {
    case 1: paged_decode_kernel<T, D, 1><<<grid, kThreads, 0, s>>>(a); break;
    case 2: paged_decode_kernel<T, D, 2><<<grid, kThreads, 0, s>>>(a); break;
    case 4: paged_decode_kernel<T, D, 4><<<grid, kThreads, 0, s>>>(a); break;
    case 8: paged_decode_kernel<T, D, 8><<<grid, kThreads, 0, s>>>(a); break;
    default: set_error("unsupported group size %d", group); return KUNSERVE_EUNSUPPORTED;
  }
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

template <typename T, int D>
int launch_merge(const int32_t* merges, int num_merge, const int32_t* q_token, const float* po,
                 const float* pl, f16* out, int64_t o_tok, int64_t o_head, int hq, hipStream_t s) {
  dim3 grid(num_merge, hq);
  decode_merge_kernel<T, D><<<grid, kWave, 0, s>>>(merges, q_token, po, pl,
                                                   reinterpret_cast<T*>(out),
                                                   o_tok, o_head, hq);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

// Partition kernel, then (for split rows) the merge, for element type T.
template <typename T>
int run_decode(const DecodeArgs& a, const kunserve_decode_plan_info& info, const int32_t* plan_dev,
               int head_dim, int num_qo_heads, dim3 grid, hipStream_t s) {
  int rc;
  switch (head_dim) {
    case 64: rc = launch_decode<T, 64>(a, info.group_size, grid, s); break;
    case 128: rc = launch_decode<T, 128>(a, info.group_size, grid, s); break;
    case 256: rc = launch_decode<T, 256>(a, info.group_size, grid, s); break;
    default: set_error("head_dim %d not compiled", head_dim); return KUNSERVE_EUNSUPPORTED;
  }
  if (rc || info.num_merge == 0) return rc;
  const int32_t* merges = plan_dev + 4 * int64_t(info.num_work);
  switch (head_dim) {
    case 64:
      return launch_merge<T, 64>(merges, info.num_merge, a.q_token, a.part_o, a.part_lse, a.out, a.o_tok,
                                 a.o_head, num_qo_heads, s);
    case 128:
      return launch_merge<T, 128>(merges, info.num_merge, a.q_token, a.part_o, a.part_lse, a.out, a.o_tok,
                                  a.o_head, num_qo_heads, s);
    default:
      return launch_merge<T, 256>(merges, info.num_merge, a.q_token, a.part_o, a.part_lse, a.out, a.o_tok,
                                  a.o_head, num_qo_heads, s);
  }
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace
}  // namespace kunserve

using namespace kunserve;

extern "C" int64_t kunserve_decode_plan_bound(const int32_t* kv_len_host, int32_t num_seqs) {
  if (num_seqs < 0 || (num_seqs > 0 && !kv_len_host)) return -1;
  int64_t parts = 0;
  for (int32_t b = 0; b < num_seqs; ++b)
    parts += std::max<int64_t>(1, ceil_div(std::max(kv_len_host[b], 0), kMinPartTokens));
  // work records (8 lanes, each at most every item) and merge records
  return 4 * (8 * parts + num_seqs);
}

extern "C" int kunserve_decode_plan(const int32_t* kv_len_host, int32_t num_seqs,
                                    int32_t num_qo_heads, int32_t num_kv_heads, int32_t num_cus,
                                    int32_t part_tokens, int32_t* plan_host,
                                    int64_t plan_capacity, kunserve_decode_plan_info* info) {
  clear_error();
  KSV_CHECK_ARG(info && plan_host, "null plan buffer or info");
  KSV_CHECK_ARG(num_seqs >= 0 && (num_seqs == 0 || kv_len_host), "bad kv_len / num_seqs");
  KSV_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads, num_kv_heads);
  for (int32_t b = 0; b < num_seqs; ++b)
    KSV_CHECK_ARG(kv_len_host[b] >= 0, "kv_len[%d] = %d < 0", b, kv_len_host[b]);
  const int group = pick_group(num_qo_heads / num_kv_heads);
  const int64_t head_groups = num_qo_heads / group;

  if (part_tokens == 0) {
    // The longest power-of-two partition whose longest work item is at most
    // 3/4 of one CU's share of the launch (a workgroup streams nearly as
    // fast alone as a CU's share of the device, so an item that long still
    // ends with the others when it starts first) and that gives every CU
    // at least 4 workgroups. Longer partitions mean fewer splits, fewer
    // partials and, once no row is split, no merge launch: the Llama-2-7B
    // decode (64 rows of lognormal(700) tokens, 32 heads) takes 136.0 us
    // per layer at 4096 (whole rows) against 138.7 at 2048, 139.0 at 1024
    // and 140.3 at 512, and the Llama-3-8B GQA and Llama-2-70B layers run
    // 1.4% and 2.4% faster at 4096 than at 2048.
    int64_t total = 0;
    int32_t max_len = 0;
    for (int32_t b = 0; b < num_seqs; ++b) {
      total += kv_len_host[b];
      max_len = std::max(max_len, kv_len_host[b]);
    }
    const int64_t cus = std::max(num_cus, 1);
    const double share = double(total) * double(head_groups) / double(cus);
    auto workgroups = [&](int64_t part) {
      int64_t n = 0;
      for (int32_t b = 0; b < num_seqs; ++b)
        n += std::max<int64_t>(1, ceil_div(kv_len_host[b], part));
      return n * head_groups;
    };
    part_tokens = kMinPartTokens;
    for (int64_t part = kMaxPartTokens; part > kMinPartTokens; part /= 2) {
      if (double(std::min<int64_t>(part, max_len)) <= 0.75 * share &&
          workgroups(part) >= 4 * cus) {
        part_tokens = int32_t(part);
        break;
      }
    }
    // A short launch (under 8 minimum partitions per CU) whose whole rows
    // already give every CU a work item, none longer than two partitions:
    // splitting would at most halve the longest item and add the merge
    // launch, which costs more than that here (single-layer batch of 8
    // rows of U[128, 512] tokens: 10.2 us unsplit against 12.2-13.2 us
    // split at 256). Keep whole rows then.
    const int64_t per = total * head_groups / (cus * 8);
    if (part_tokens == kMinPartTokens && per < kMinPartTokens &&
        int64_t(num_seqs) * head_groups >= cus && max_len <= 2 * part_tokens) {
      while (part_tokens < max_len && part_tokens < kMaxPartTokens) part_tokens *= 2;
    }
  }
  KSV_CHECK_ARG(part_tokens >= kMinPartTokens && part_tokens <= kMaxPartTokens &&
                    part_tokens % 64 == 0,
                "part_tokens %d must be a multiple of 64 in [%d, %d]", part_tokens,
                kMinPartTokens, kMaxPartTokens);

  // Work items: (seq, begin, end, slot). Full partitions first, then tails
  // by decreasing length, so the longest items start first.
  struct Item { int32_t seq, b, e, slot; };
  std::vector<Item> items;
  std::vector<int32_t> merges;
  int32_t slots = 0;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t len = kv_len_host[b];
    const int32_t n = std::max<int32_t>(1, int32_t(ceil_div(len, part_tokens)));
    if (n == 1) {
      items.push_back({b, 0, len, -1});
    } else {
      merges.insert(merges.end(), {b, slots, n, 0});
      for (int32_t j = 0; j < n; ++j)
        items.push_back({b, j * part_tokens, std::min(len, (j + 1) * part_tokens), slots + j});
      slots += n;
    }
  }
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& x, const Item& y) { return (x.e - x.b) > (y.e - y.b); });
  // One lane per XCD, dealt longest first to the lane that would finish it
  // first at that XCD's streaming rate. On MI355X the odd XCDs stream decode
  // about 7% slower than the even ones (10.8 against 11.6 tokens per us per
  // workgroup at the Llama-2-7B shape, the same on every layer and with the
  // items rotated across XCDs: a property of the XCD, not of the data), so
  // an even share left them finishing 5-7 us after the even XCDs. A
  // workgroup's start costs about 32 tokens of streaming.
  constexpr double kXcdRate[kXcds] = {1.0, 0.93, 1.0, 0.93, 1.0, 0.93, 1.0, 0.93};
  constexpr double kItemStartTokens = 32.0;
  std::vector<Item> lanes[kXcds];
  double load[kXcds] = {};
  for (const Item& it : items) {
    const double cost = double(it.e - it.b) + kItemStartTokens;
    int best = 0;
    for (int x = 1; x < kXcds; ++x)
      if ((load[x] + cost) / kXcdRate[x] < (load[best] + cost) / kXcdRate[best]) best = x;
    lanes[best].push_back(it);
    load[best] += cost;
  }
  size_t depth = 0;
  for (const auto& l : lanes) depth = std::max(depth, l.size());
  const int64_t need = 4 * int64_t(kXcds) * int64_t(depth) + int64_t(merges.size());
  if (need > plan_capacity) {
    set_error("plan needs %lld ints, capacity %lld", (long long)need, (long long)plan_capacity);
    return KUNSERVE_ENOSPC;
  }
  int32_t* p = plan_host;
  for (size_t r = 0; r < depth; ++r)
    for (int x = 0; x < kXcds; ++x) {
      const Item it = r < lanes[x].size() ? lanes[x][r] : Item{-1, 0, 0, -1};
      *p++ = it.seq;
      *p++ = it.b;
      *p++ = it.e;
      *p++ = it.slot;
    }
  std::copy(merges.begin(), merges.end(), p);
  info->num_work = int32_t(kXcds * depth);
  info->num_merge = int32_t(merges.size() / 4);
  info->num_slots = slots;
  info->part_tokens = part_tokens;
  info->group_size = group;
  info->plan_ints = int32_t(need);
  return KUNSERVE_OK;
}

extern "C" int64_t kunserve_decode_workspace_bytes(const kunserve_decode_plan_info* info,
                                                   int32_t num_qo_heads, int32_t head_dim) {
  if (!info || num_qo_heads <= 0 || head_dim <= 0) return -1;
  const int64_t slots = info->num_slots;
  return slots * num_qo_heads * (int64_t(head_dim) + 1) * int64_t(sizeof(float));
}

extern "C" int kunserve_paged_decode(const kunserve_kv_pool* pool, int32_t layer,
                                     const kunserve_page_table* table,
                                     const int32_t* q_token_dev,
                                     const kunserve_tensor3* q, kunserve_tensor3* out,
                                     int32_t num_qo_heads, float sm_scale,
                                     const int32_t* plan_dev,
                                     const kunserve_decode_plan_info* info, void* workspace_dev,
                                     int64_t workspace_bytes, kunserve_stream_t stream) {
  clear_error();
  int rc = check_pool(pool, true);
  if (rc) return rc;
  KSV_CHECK_ARG(table && q && out && info, "null argument");
  KSV_CHECK_ARG(layer >= 0 && layer < pool->num_layers, "layer %d outside [0, %d)", layer,
                pool->num_layers);
  KSV_CHECK_ARG(std::isfinite(sm_scale) && sm_scale > 0.f,
                "sm_scale %g must be finite and positive", double(sm_scale));
  KSV_CHECK_ARG(num_qo_heads > 0 && num_qo_heads % pool->num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads,
                pool->num_kv_heads);
  const int ratio = num_qo_heads / pool->num_kv_heads;
  KSV_CHECK_ARG(info->group_size >= 1 && ratio % info->group_size == 0,
                "plan group size %d does not divide the GQA ratio %d", info->group_size, ratio);
  if (info->num_work == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(plan_dev && table->indptr_dev && table->indices_dev, "null plan or table");
  KSV_CHECK_ARG(q->data && out->data && aligned16(q->data) &&
                    (q->token_stride % 8) == 0 && (q->head_stride % 8) == 0,
                "q must be 16-byte aligned with strides that are multiples of 8");
  const int64_t ws_need = kunserve_decode_workspace_bytes(info, num_qo_heads, pool->head_dim);
  if (info->num_slots > 0 && (workspace_bytes < ws_need || !workspace_dev)) {
    set_error("decode workspace holds %lld bytes, %lld needed", (long long)workspace_bytes,
              (long long)ws_need);
    return KUNSERVE_ENOSPC;
  }
  DecodeArgs a{};
  a.q_token = q_token_dev;
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
  a.work = plan_dev;
  float* ws = static_cast<float*>(workspace_dev);
  a.part_o = ws;
  a.part_lse = ws ? ws + int64_t(info->num_slots) * num_qo_heads * pool->head_dim : nullptr;
  a.num_qo_heads = num_qo_heads;
  a.ratio = ratio;
  a.scale_log2 = sm_scale * 1.4426950408889634f;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // One dimension, mapped to (record, head group) by decode_work: on every
  // XCD the dispatch order is its lane's longest-first order (a launch ends
  // on short items), with an item's head groups, which read the same pages,
  // back to back.
  a.head_groups = num_qo_heads / info->group_size;
  a.num_work = info->num_work;
  const int64_t nblocks = 8 * ceil_div(info->num_work, 8) * a.head_groups;
  KSV_CHECK_ARG(nblocks < (int64_t(1) << 31), "decode grid of %lld workgroups is too large",
                (long long)nblocks);
  const dim3 grid(static_cast<unsigned>(nblocks));
  if (pool->dtype == KUNSERVE_DTYPE_BF16)
    return run_decode<bf16>(a, *info, plan_dev, pool->head_dim, num_qo_heads, grid, s);
  return run_decode<f16>(a, *info, plan_dev, pool->head_dim, num_qo_heads, grid, s);
}

// ------------------------------------------------ access-pattern calibration
// kunserve_decode_slab_probe reads a decode launch's K/V slabs (one page's
// tokens of one head: page_size x head_dim elements, contiguous) in the
// partition kernel's shape, with the slab offsets precomputed and no
// arithmetic on the data: workgroup i x heads + h reads item i's slabs of
// head h, its 4 waves striding them, two slabs in flight per wave, 1 KiB per
// load instruction, non-temporal. Each workgroup XORs what it read into
// sink[workgroup], so a test can check the bytes.
namespace kunserve {
namespace {

constexpr int kMaxSlabLoads = 16;   // 1 KiB loads per slab and tensor (slabs up to 16 KiB)

template <int NL>
__device__ __forceinline__ void probe_slab(const char* k, const char* v, int64_t off, int lane,
                                           u32x4 (&x)[2 * NL]) {
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    x[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k + off + i * 1024 + lane * 16));
    x[NL + i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(v + off + i * 1024 + lane * 16));
  }
}

template <int NL>
__global__ __launch_bounds__(kThreads) void decode_slab_probe_kernel(
    const char* k, const char* v, const int64_t* offs, const int32_t* counts, int max_slabs,
    int64_t head_bytes, int heads, uint32_t* sink) {
  __shared__ int64_t s_off[kMaxPartPages];
  __shared__ uint32_t s_x[kWaves];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // The decode's dispatch order: an item's heads on one XCD, items of the
  // 8 XCD lanes interleaved.
  const int j = int(blockIdx.x) >> 3;
  const int local = j / heads;
  const int head = j - local * heads;
  const int item = 8 * local + (int(blockIdx.x) & 7);
  const int n = min(counts[item], max_slabs);
  // The item's offsets are staged in LDS, as the decode stages its page ids.
  const int64_t* o = offs + int64_t(item) * max_slabs;
  for (int i = threadIdx.x; i < n; i += kThreads) s_off[i] = o[i];
  __syncthreads();
  const int64_t hoff = int64_t(head) * head_bytes;
  u32x4 acc = {0u, 0u, 0u, 0u};
  u32x4 a[2 * NL], b[2 * NL];
  int s = wave;
  if (s < n) probe_slab<NL>(k, v, s_off[s] + hoff, lane, a);
  while (s < n) {
    const int s2 = s + kWaves;
    if (s2 < n) probe_slab<NL>(k, v, s_off[s2] + hoff, lane, b);
#pragma unroll
    for (int i = 0; i < 2 * NL; ++i) acc ^= a[i];
    s = s2;
    if (s >= n) break;
    const int s3 = s + kWaves;
    if (s3 < n) probe_slab<NL>(k, v, s_off[s3] + hoff, lane, a);
#pragma unroll
    for (int i = 0; i < 2 * NL; ++i) acc ^= b[i];
    s = s3;
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= uint32_t(__shfl_xor(int(x), off));
  if (lane == 0) s_x[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) r ^= s_x[w];
    sink[item * heads + head] = r;
  }
}

}  // namespace
}  // namespace kunserve

extern "C" int kunserve_decode_slab_probe(const void* k_dev, const void* v_dev,
                                          const int64_t* slab_offsets_dev,
                                          const int32_t* counts_dev, int32_t num_items,
                                          int32_t max_slabs, int64_t head_stride_bytes,
                                          int32_t num_heads, int32_t slab_bytes,
                                          uint32_t* sink_dev, kunserve_stream_t stream) {
  using namespace kunserve;
  clear_error();
  KSV_CHECK_ARG(k_dev && v_dev && slab_offsets_dev && counts_dev && sink_dev, "null argument");
  KSV_CHECK_ARG(aligned16(k_dev) && aligned16(v_dev), "pools must be 16-byte aligned");
  KSV_CHECK_ARG(num_items >= 0 && num_items % 8 == 0 && max_slabs > 0 &&
                    max_slabs <= kMaxPartPages && num_heads > 0 && head_stride_bytes >= 0,
                "bad item (a multiple of 8), slab (at most %d) or head count", kMaxPartPages);
  KSV_CHECK_ARG(slab_bytes > 0 && slab_bytes % 1024 == 0 && slab_bytes / 1024 <= kMaxSlabLoads,
                "slab_bytes %d must be a multiple of 1024 up to %d", slab_bytes,
                kMaxSlabLoads * 1024);
  KSV_CHECK_ARG(int64_t(num_items) * num_heads < (int64_t(1) << 31), "too many workgroups");
  if (num_items == 0) return KUNSERVE_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const char* k = static_cast<const char*>(k_dev);
  const char* v = static_cast<const char*>(v_dev);
  const dim3 grid(static_cast<unsigned>(int64_t(num_items) * num_heads));
  switch (slab_bytes / 1024) {
    case 1: decode_slab_probe_kernel<1><<<grid, kThreads, 0, s>>>(k, v, slab_offsets_dev, counts_dev, max_slabs, head_stride_bytes, num_heads, sink_dev); break;
    case 2: decode_slab_probe_kernel<2><<<grid, kThreads, 0, s>>>(k, v, slab_offsets_dev, counts_dev, max_slabs, head_stride_bytes, num_heads, sink_dev); break;
    case 4: decode_slab_probe_kernel<4><<<grid, kThreads, 0, s>>>(k, v, slab_offsets_dev, counts_dev, max_slabs, head_stride_bytes, num_heads, sink_dev); break;
    case 8: decode_slab_probe_kernel<8><<<grid, kThreads, 0, s>>>(k, v, slab_offsets_dev, counts_dev, max_slabs, head_stride_bytes, num_heads, sink_dev); break;
    case 16: decode_slab_probe_kernel<16><<<grid, kThreads, 0, s>>>(k, v, slab_offsets_dev, counts_dev, max_slabs, head_stride_bytes, num_heads, sink_dev); break;
    default: set_error("slab_bytes %d: 1, 2, 4, 8 or 16 KiB", slab_bytes); return KUNSERVE_EINVAL;
  }
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

// ------------------------------------------------ decode without allocation
// kunserve_paged_decode_noalloc keeps the split partials in `scratch`, a
// file-scope device array of kNoAllocScratchBytes that every device the
// library runs on holds until the process ends. In host code `scratch` is
// only a stand-in for the symbol: its device address, one per device, comes
// from hipGetSymbolAddress with that device current, and only that address
// is ever handed to a kernel.
namespace kunserve {
namespace {

constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_ptr;   // by device ordinal

// Device address of `scratch` on `device`, looked up once per device.
int scratch_address(int device, void** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (device >= int(g_scratch_ptr.size())) g_scratch_ptr.resize(device + 1, nullptr);
  if (!g_scratch_ptr[device]) {
    int current = 0;
    KSV_CHECK_HIP(hipGetDevice(&current));
    if (current != device) KSV_CHECK_HIP(hipSetDevice(device));
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current != device) KSV_CHECK_HIP(hipSetDevice(current));
    if (e != hipSuccess || !ptr) {
      set_error("hipGetSymbolAddress(scratch) on device %d failed: %s", device,
                hipGetErrorString(e));
      return KUNSERVE_EHIP;
    }
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return KUNSERVE_OK;
}

}  // namespace
}  // namespace kunserve

extern "C" int64_t kunserve_paged_decode_noalloc_max_bytes(void) {
  return kunserve::kNoAllocScratchBytes;
}

extern "C" int kunserve_paged_decode_noalloc(const kunserve_kv_pool* pool, int32_t layer,
                                             const kunserve_page_table* table,
                                             const int32_t* q_token_dev,
                                             const kunserve_tensor3* q, kunserve_tensor3* out,
                                             int32_t num_qo_heads, float sm_scale,
                                             const int32_t* plan_dev,
                                             const kunserve_decode_plan_info* info,
                                             kunserve_stream_t stream) {
  using namespace kunserve;
  clear_error();
  int rc = check_pool(pool, true);
  if (rc) return rc;
  KSV_CHECK_ARG(info != nullptr, "null plan info");
  const int64_t need = kunserve_decode_workspace_bytes(info, num_qo_heads, pool->head_dim);
  KSV_CHECK_ARG(need >= 0, "bad plan or head counts");
  if (need > kNoAllocScratchBytes) {
    set_error("decode partials need %lld bytes, more than the %lld bytes of the static "
              "scratch of kunserve_paged_decode_noalloc; use kunserve_paged_decode with a "
              "workspace", (long long)need, (long long)kNoAllocScratchBytes);
    return KUNSERVE_ENOSPC;
  }
  void* ws = nullptr;
  if (need > 0) {
    int device = 0;
    if (stream) {
      KSV_CHECK_HIP(hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &device));
    } else {
      KSV_CHECK_HIP(hipGetDevice(&device));
    }
    rc = scratch_address(device, &ws);
    if (rc) return rc;
  }
  return kunserve_paged_decode(pool, layer, table, q_token_dev, q, out, num_qo_heads, sm_scale,
                               plan_dev, info, ws, need > 0 ? kNoAllocScratchBytes : 0, stream);
}
