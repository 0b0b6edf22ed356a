// Chunked-prefill attention with K/V append into pages (prefill rows of
// LlamaOp.pforward, kunserve/worker.py:298-312; chunk bounds
// kunserve/request.py:368-391,428-437; first index kunserve/request.py:447-462).
//
// Append: HBM-bound scatter of the new tokens' K/V rows into their pages.
//
// Attention: flash-attention style on fp16 or bf16 MFMA
// (v_mfma_f32_32x32x16_f16 / _bf16, gfx950), fp32 accumulation and online
// softmax; kernels are templates over the element type.
//  * Every compute wave owns 32 query rows of one (sequence, q head).
//    Loader waves gather 64-token K/V tiles from the pages into LDS: K
//    row-major, V transposed (one row per dim), so that both operands are
//    16-byte reads; page positions are looked up one tile ahead.
//  * head_dim 64 and 128 (paged_prefill_ws_kernel): 8 compute waves (256
//    rows, two per SIMD) and 4 loader waves; a ring of 2 K and 3 V buffers.
//  * head_dim 256 (paged_prefill_kernel): 4 compute waves (128 rows, one
//    per SIMD) and 4 loader waves; 2 K and 2 V buffers, one barrier per
//    tile; each tile's two 32-token halves run as a pipeline.
//  * S^T = K.Q^T is computed so that the accumulator layout (one query row
//    per lane column) is directly the B operand of O^T = V^T.P^T: the
//    probabilities never leave registers.
//  * Causal masking only on tiles that cross a wave's diagonal; tiles past
//    a wave's last visible position skip the math.
//  * The plan places the workgroups that read the same K/V (same sequence
//    and KV head) back to back on one XCD so that they share its L2.
//  * Steps with too few q tiles to fill the device split each tile's KV
//    range over several workgroups; those write fp32 partials (O, running
//    max, sum) and a merge kernel combines them in split order.
#include <algorithm>
#include <cmath>
#include <vector>

#include "common.hpp"

namespace kunserve {
namespace {

constexpr int kTileKV = 64;           // kv tokens per iteration
constexpr int kVtPitch = kTileKV;     // halves per row of the transposed V tile
constexpr int kXcds = 8;              // MI355X: workgroup i runs on XCD i % 8

// Geometry of the attention kernel for one head_dim. Every compute wave
// owns 32 query rows (the 32x32 MFMA's columns). Up to head_dim 128 a
// workgroup is 8 waves, two per SIMD, each computing and gathering; at 256
// it is 4 compute waves, one per SIMD, since the O accumulators and Q
// operands of a wave then take 192 registers, and 4 loader waves, one per
// SIMD, that only gather K/V tiles into LDS.
template <int D>
struct Geom {
  static_assert(D == 64 || D == 128 || D == 256, "prefill head_dim is 64, 128 or 256");
  static constexpr int kComputeWaves = D <= 128 ? 8 : 4;
  static constexpr int kLoadWaves = D <= 128 ? 0 : 4;
  static constexpr int kWaves = kComputeWaves + kLoadWaves;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kTileQ = 32 * kComputeWaves;   // query rows per workgroup
  static constexpr int kSteps = D / 16;        // 16-dim k-steps of S = K.Q^T
  static constexpr int kBlocks = D / 32;       // 32-dim blocks of O
  static constexpr int kKPitch = D + 8;        // halves per K row
  static constexpr int kKHalves = kTileKV * kKPitch;
  static constexpr int kVtHalves = D * kVtPitch;
  // Gather units (4 consecutive tokens x one 16-byte chunk of K or V) per
  // lane of a gathering wave: 64 and 128: one (waves 0-1 / 0-3 gather V,
  // 2-3 / 4-7 gather K); 256: four (every loader wave two chunks of V and
  // two of K).
  static constexpr int kUnits = D == 256 ? 4 : 1;
  // Gather register sets: two (the tile after next in flight while the next
  // waits to be stashed) up to 128; one at 256, where the loader waves
  // fetch tile it + 2 as soon as tile it + 1 has left the registers, a whole
  // tile of math (twice that of 128) ahead of its stash.
  static constexpr int kRegSets = D <= 128 ? 2 : 1;
};

constexpr int tile_q_for(int head_dim) { return head_dim <= 128 ? 256 : 128; }
static_assert(tile_q_for(64) == Geom<64>::kTileQ && tile_q_for(128) == Geom<128>::kTileQ &&
                  tile_q_for(256) == Geom<256>::kTileQ,
              "the plan's tile is the kernel's");

struct PrefillArgs {
  const f16* q;
  int64_t q_tok, q_head;
  f16* out;
  int64_t o_tok, o_head;
  const f16* k;   // pool K at the layer
  const f16* v;
  int64_t head_stride;
  uint32_t page_stride, token_stride;   // checked on the host to fit 32 bits
  int32_t num_pages;
  int32_t page_shift;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* kv_len;
  const int32_t* q_indptr;
  const int32_t* q_start; // null, or [num_seqs]: first token of each row in q and out
  const int32_t* tiles;   // [num_tiles][kRec]: see kRec
  float* part_o;          // [slots][tile_q][head_dim] split partials, normalised
  float* part_ml;         // [slots][tile_q][2] running max (log2 units), sum
  int32_t ratio;
  float scale_log2;
};

// Plan record of one workgroup: seq (-1: padding), first q row, q head,
// KV range [kv_lo, kv_hi) it attends over, partial slot (-1: writes out).
constexpr int kRec = 6;
// Merge record: seq, first q row, q head, first slot, number of splits.
constexpr int kMergeRec = 5;

// LDS layouts; every operand address is a per-lane base plus an immediate
// offset. Bank behaviour was measured on gfx950 with SQ_LDS_BANK_CONFLICT:
// 8-byte stores go 16 lanes per cycle over 32 banks; the 16-byte accesses
// below measured conflict-free (16-byte reads follow no simple lane-group
// model, so layouts were chosen by measurement).
// K tile: row-major [token][dim], rows head_dim + 8 halves apart (68
//   dwords at 128); operand reads (row 32 mt + r, one 16-byte chunk) and the
//   gather's 16-byte row stores are conflict-free.
// V tile: transposed, row d holds dim d of the tile's 64 tokens, rows 128
//   bytes apart, so the V^T operands are plain 16-byte reads (the gfx950
//   transposing read, ds_read_b64_tr_b16, moves a quarter of the bytes per
//   cycle, and every wave reads the whole tile). Columns follow the P^T
//   operand: within each 16 tokens, token 8a + 4h + b sits at column
//   8h + 4a + b, so the 8 tokens one lane's operand needs are one 16-byte
//   chunk. Chunk c of row d is stored at chunk c ^ ((d ^ (d >> 3)) & 7):
//   conflict-free for both the operand reads and the gather's 8-byte stores
//   (a store pass, 16 lanes, covers 8 dims 8 apart x both halves of a chunk).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Gather layout. A lane moves 4 consecutive tokens 16 g + 8 a + 4 h + i
// (i < 4) of 16-byte chunks c of K or V: token group g (0..3), a and h pick
// the lane's 4 tokens within the group. Lane bits: c = l & 7 and a = bit 3
// always, so that every 16 lanes cover both halves a of 8 chunks (the
// transposed stores' conflict-free pass); then, at head_dim 64, h = bit 4
// and g = 2 w + bit 5 (wave w of a pair); at 128 and 256, c |= bit 4 << 3,
// h = bit 5 and g = the wave's group (256: chunks 16..31 as a second
// unit). The tokens are 4-aligned, so (page_size >= 4) one page holds them.
struct GatherLane {
  int g, c, a, h;
};
template <int D>
__device__ __forceinline__ GatherLane gather_lane(int group, int lane) {
  if constexpr (D == 64)
    return {2 * group + (lane >> 5), lane & 7, (lane >> 3) & 1, (lane >> 4) & 1};
  else
    return {group, (lane & 7) | (((lane >> 4) & 1) << 3), (lane >> 3) & 1, lane >> 5};
}

// Transposed store of dims 2 part, 2 part + 1 of chunk c of a gathering
// lane's 4 tokens (x[i]: token i, 8 dims) into the V^T buffer buf. Dim
// 8 c + e of token group g is row 8 c + e, logical chunk 2 g + h, stored at
// chunk (2 g + h) ^ (c & 7) ^ e, at half 4 a of it. v_perm builds each
// dword from two tokens' dwords; its selector byte 0x0c yields a zero
// byte, which zeroes the tokens from nok on.
template <typename T>
__device__ __forceinline__ void vt_store(T* buf, const GatherLane& gl, int c,
                                         const typename Vec<T>::v8 (&x)[4], int part, int nok) {
  const int row0 = 8 * c * kVtPitch + 4 * gl.a;
  const int chunk0 = (2 * gl.g + gl.h) ^ (c & 7);
  const uint32_t z01 = (nok < 1 ? 0x0000ffffu : 0u) | (nok < 2 ? 0xffff0000u : 0u);
  const uint32_t z23 = (nok < 3 ? 0x0000ffffu : 0u) | (nok < 4 ? 0xffff0000u : 0u);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int e = 2 * part + half;
    const uint32_t sel = half ? 0x07060302u : 0x05040100u;   // high / low halves
    const uint32_t s01 = (sel & ~z01) | (0x0c0c0c0cu & z01);
    const uint32_t s23 = (sel & ~z23) | (0x0c0c0c0cu & z23);
    const u32x2 d = {__builtin_amdgcn_perm(__builtin_bit_cast(u32x4, x[1])[part],
                                           __builtin_bit_cast(u32x4, x[0])[part], s01),
                     __builtin_amdgcn_perm(__builtin_bit_cast(u32x4, x[3])[part],
                                           __builtin_bit_cast(u32x4, x[2])[part], s23)};
    *reinterpret_cast<u32x2*>(buf + row0 + e * kVtPitch + 8 * (chunk0 ^ e)) = d;
  }
}

// V^T operand (ks, dt) of lane (r, h): row d = 32 dt + r, logical chunk
// 2 ks + h, stored at chunk (2 ks + h) ^ ((d ^ (d >> 3)) & 7)
// = (2 ks ^ 4 (dt & 1)) ^ (h ^ (r & 7) ^ (r >> 3)) (r >> 3 < 4, so d >> 3
// adds no carry into bit 2): one of four per-lane bases, j = ks ^ 2 (dt & 1),
// plus an immediate offset.
struct VtBases {
  int b[4];
};
__device__ __forceinline__ VtBases vt_operand_bases(int lane) {
  const int r = lane & 31, h = lane >> 5;
  const int s = h ^ (r & 7) ^ (r >> 3);
  VtBases v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v.b[j] = r * kVtPitch + 8 * ((2 * j) ^ s);
  return v;
}
__device__ __forceinline__ int vt_operand_base_index(int ks, int dt) { return ks ^ (2 * (dt & 1)); }
__device__ __forceinline__ int vt_operand_offset(int dt) { return 32 * dt * kVtPitch; }

// Where a gathering lane's 4 tokens of the tile at kv token tok0 are:
// element offset in a layer and how many of them hold data (0 on a page id
// outside the pool, else those before kv_end). Ids outside the pool read
// page 0, so every load is in bounds with no select: K rows past kv_end or
// on a bad page are masked out of the scores, V rows are zeroed by the
// stash (a zero probability times whatever such a row holds could be NaN).
struct TileAt {
  uint64_t off;
  int nok;
};
__device__ __forceinline__ TileAt tile_at(int p, int tok0, int kv_end, int num_pages,
                                          uint32_t page_stride, uint32_t token_stride,
                                          int page_mask, int dim) {
  const bool pg_ok = uint32_t(p) < uint32_t(num_pages);
  return TileAt{uint64_t(uint32_t(pg_ok ? p : 0)) * page_stride +
                    (uint32_t(tok0 & page_mask) * token_stride + dim),
                pg_ok ? max(0, min(4, kv_end - tok0)) : 0};
}

// Page ids a workgroup stages in LDS (rows up to 32768 tokens at page 16).
constexpr int kMaxStagedPages = 2048;

// STAGED: the row's page ids are copied to LDS once, so the tile gathers
// issue only K/V loads; waiting for an older tile's data then leaves the
// newer tile's loads in flight. Rows with more pages than fit use the
// global-lookup variant (same results).
template <typename T, int D, bool STAGED>
__global__ __launch_bounds__(Geom<D>::kThreads) void paged_prefill_kernel(PrefillArgs a) {
  typedef typename Vec<T>::v8 V8;
  typedef typename Vec<T>::v4 V4;
  typedef Geom<D> G;
  __shared__ int s_pg[STAGED ? kMaxStagedPages : 1];
  __shared__ int s_bad[G::kWaves];
  __shared__ __attribute__((aligned(16))) T sK[2 * G::kKHalves];
  __shared__ __attribute__((aligned(16))) T sVt[2 * G::kVtHalves];

  const int32_t* item = a.tiles + kRec * blockIdx.x;
  const int seq = item[0];
  if (seq < 0) return;   // padding workgroup (uniform: no barrier reached)
  const int q0 = item[1];
  const int hq = item[2];
  const int kv_lo = item[3];   // a multiple of kTileKV
  const int kv_hi = item[4];
  const int slot = item[5];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // scalar: gather role branches on it
  const int r = lane & 31;       // query row within the wave / MFMA column
  const int h = lane >> 5;       // MFMA k-half

  const int hkv = hq / a.ratio;
  const int qb = a.q_indptr[seq];
  const int q_len = a.q_indptr[seq + 1] - qb;
  const int qt = a.q_start ? a.q_start[seq] : qb;   // the row's first token of q and out
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
  const int kv_end = min(prefix + min(q0 + G::kTileQ, q_len), kv_hi);   // exclusive
  const int ntiles = (kv_end + kTileKV - 1) / kTileKV;   // tiles [kv_lo / kTileKV, ntiles)
  const int pg_lo = kv_lo >> a.page_shift;   // first staged page
  // Stage (or, for rows with too many pages, only scan) the page ids of
  // [kv_lo, kv_end). Whether any of them is outside the pool is voted per
  // wave: only then do the scores need a per-page mask, which drops the
  // tokens of such pages from the softmax.
  bool any_bad = false;
  {
    const int npg = kv_end > kv_lo ? ((kv_end - 1) >> a.page_shift) + 1 - pg_lo : 0;
    bool bad_id = false;
    for (int i = threadIdx.x; i < npg; i += G::kThreads) {
      const int p = pages[pg_lo + i];
      const bool ok = p >= 0 && p < a.num_pages;
      if constexpr (STAGED) s_pg[i] = ok ? p : -1;
      bad_id |= !ok;
    }
    const bool wave_bad = __any(bad_id);
    if ((threadIdx.x & 63) == 0) s_bad[threadIdx.x >> 6] = wave_bad;
    __syncthreads();
    int bad = 0;
#pragma unroll
    for (int wv = 0; wv < G::kWaves; ++wv) bad |= s_bad[wv];
    any_bad = __builtin_amdgcn_readfirstlane(bad) != 0;   // the same in every lane
  }
  // Whether kv token `tok` (< kv_end) lies on an out-of-range page.
  auto bad_page = [&](int tok) {
    const int p = STAGED ? s_pg[(tok >> a.page_shift) - pg_lo] : pages[tok >> a.page_shift];
    return uint32_t(p) >= uint32_t(a.num_pages);
  };

  f32x16 o[G::kBlocks];
#pragma unroll
  for (int i = 0; i < G::kBlocks; ++i) o[i] = f32x16{};
  float m = -1.0e30f;   // running max of this row, in scaled (log2) units
  float lsum = 0.f;     // this lane's share of the row sum (other half: lane ^ 32)

  const f16* kbase = a.k + int64_t(hkv) * a.head_stride;
  const f16* vbase = a.v + int64_t(hkv) * a.head_stride;

  // Tile registers: two sets, so that the gather of tile n + 2 is in flight
  // while tile n is computed and tile n + 1 waits to be parked in LDS. One
  // tile's loads take about one HBM round trip, longer than a tile's math.
  // Gather roles (Geom::kUnits): at head_dim 64 waves 0-1 gather V and 2-3
  // K; at 128 waves 0-3 V and 4-7 K; at 256 every loader wave both, two
  // chunks of each. The tile position of a gather is looked up one iteration ahead
  // (at), so no lookup latency sits in front of the loads. Every wave
  // issues its loads unconditionally (at 64, waves 4-7 repeat those of
  // waves 0-3, which the CU's cache serves, and do not stash them): a
  // branch around loads makes the compiler wait for all loads in flight,
  // the ones just issued too, wherever the branch joins.
  constexpr int kGatherWaves = D == 64 ? 4 : G::kWaves;
  const bool stashes = kGatherWaves == G::kWaves || wave < kGatherWaves;
  const int gw = wave % kGatherWaves;
  const bool gather_v = D == 256 || gw < kGatherWaves / 2;   // the first unit's tensor
  const GatherLane gl = gather_lane<D>(D == 256 ? wave - G::kComputeWaves : gw % (kGatherWaves / 2), lane);
  const int ld_t = 16 * gl.g + 8 * gl.a + 4 * gl.h;
  const int ld_c = 8 * gl.c;
  // Unit u: tensor (V for the first half at 256), chunk gl.c + 16 (u & 1) at 256.
  auto unit_v = [&](int u) { return D == 256 ? u < 2 : gather_v; };
  auto unit_c = [&](int u) { return gl.c + (D == 256 ? 16 * (u & 1) : 0); };
  struct Regs {
    V8 x[G::kUnits][4];
    int nok;
  };
  TileAt at;
  auto read_ids = [&](int n0) {
    const int tok = n0 + ld_t;
    const int t = max(kv_lo, min(tok, kv_end - 1));   // clamped into the staged range
    const int p = STAGED ? s_pg[(t >> a.page_shift) - pg_lo] : pages[t >> a.page_shift];
    at = tile_at(p, tok, kv_end, a.num_pages, a.page_stride, a.token_stride, page_mask, ld_c);
  };
  auto fetch = [&](Regs& rg) {
#pragma unroll
    for (int u = 0; u < G::kUnits; ++u) {
      const f16* base = (unit_v(u) ? vbase : kbase) + at.off + 8 * (unit_c(u) - gl.c);
#pragma unroll
      for (int i = 0; i < 4; ++i) rg.x[u][i] = load_v8<T>(base + int64_t(i) * a.token_stride);
    }
    rg.nok = at.nok;
  };
  auto stash = [&](int buf, const Regs& rg) {
    if (!stashes) return;
#pragma unroll
    for (int u = 0; u < G::kUnits; ++u) {
      if (unit_v(u)) {
#pragma unroll
        for (int part = 0; part < 4; ++part)
          vt_store<T>(sVt + buf * G::kVtHalves, gl, unit_c(u), rg.x[u], part, rg.nok);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<V8*>(&sK[buf * G::kKHalves + (ld_t + i) * G::kKPitch + 8 * unit_c(u)]) =
              rg.x[u][i];
      }
    }
  };

  // Q as the B operand of S^T = K.Q^T: step s covers dims 16s + 8h .. +8.
  // Loaded with no branch: a row past q_len reads the sequence's first row
  // instead (its scores stay in its own lane column, and it writes no
  // output).
  V8 qf[G::kSteps];
  auto qf_load = [&]() {
    const f16* qp = a.q + int64_t(qt + (row_ok ? qrow : 0)) * a.q_tok + int64_t(hq) * a.q_head;
#pragma unroll
    for (int s = 0; s < G::kSteps; ++s) qf[s] = load_v8<T>(qp + 16 * s + 8 * h);
  };

  // Per-lane LDS bases; each operand read adds a compile-time offset.
  // K A operand (S^T = K.Q^T): row 32 mt + r, dims 16 s + 8 h .. +8.
  const int kb0 = r * G::kKPitch + 8 * h;
  const VtBases vb = vt_operand_bases(lane);

  // A tile is two 32-token halves. The score MFMAs of the second half are
  // issued before the first half's max, and the first half's P.V before the
  // second half's max, so that with one wave per SIMD the matrix cores have
  // work while the wave runs each half's softmax.
  auto half_scores = [&](int buf, int hh) {
    const T* kt = sK + buf * G::kKHalves + kb0 + 32 * hh * G::kKPitch;
    f32x16 sv = mfma32(*reinterpret_cast<const V8*>(kt), qf[0], f32x16{});
#pragma unroll
    for (int st = 1; st < G::kSteps; ++st)
      sv = mfma32(*reinterpret_cast<const V8*>(kt + 16 * st), qf[st], sv);
    return sv;
  };
  // Masks (on tiles that need them) and the row max, in log2 units, of half
  // hh of the tile at n0. Lane (r, h) holds tokens n0 + 32 hh + 8 (v / 4) +
  // 4 h + v % 4 of query row r; lanes r and r + 32 hold the row's two halves.
  auto half_max = [&](f32x16& sv, int n0, int hh, bool masked) {
    float mx = -INFINITY;
    if (masked) {
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        // The 4 tokens of a group share one page (page_size >= 4).
        const int tok0 = n0 + 32 * hh + 8 * v4 + 4 * h;
        const bool skip = any_bad && tok0 < kv_end && bad_page(tok0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * v4 + e;
          const int tok = tok0 + e;
          if (skip || tok > qpos || tok >= kvl) sv[v] = -INFINITY;
          mx = fmaxf(mx, sv[v]);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sv[v]);
    }
    return fmaxf(mx, __shfl_xor(mx, 32)) * a.scale_log2;
  };
  // Lazy running max: move it only when a half's max exceeds it by more
  // than 8 (log2 units). Probabilities then stay <= 2^8, far inside the
  // fp16 range, and the O rescale is skipped unless some row of the wave
  // moved.
  auto rescale = [&](float mx) {
    if (__any(mx > m + 8.f)) {
      const float m_new = mx > m + 8.f ? mx : m;
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < G::kBlocks; ++dt) o[dt] *= alpha;
    }
  };
  // P^T as B operands: k-step kk covers tokens 16 kk + 4h + {0..3} and
  // 16 kk + 8 + 4h + {0..3} of the half, i.e. accumulator entries 8 kk + e.
  auto probs = [&](const f32x16& sv, V8 (&pb)[2]) {
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = fast_exp2(fmaf(sv[v], a.scale_log2, -m));
      ps += p;
      pb[v >> 3][v & 7] = T(p);
    }
    lsum += ps;
  };
  // O^T[dims, rows] += V^T[dims, tokens] . P^T[tokens, rows] over the half's
  // k-steps 2 hh and 2 hh + 1 of the V^T tile.
  auto pv = [&](int buf, int hh, const V8 (&pb)[2]) {
    const T* vt = sVt + buf * G::kVtHalves;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ks = 2 * hh + kk;
#pragma unroll
      for (int dt = 0; dt < G::kBlocks; ++dt) {
        const V8 va = *reinterpret_cast<const V8*>(vt + vb.b[vt_operand_base_index(ks, dt)] +
                                                    vt_operand_offset(dt));
        o[dt] = mfma32(va, pb[kk], o[dt]);
      }
    }
  };

  auto compute = [&](int buf, int n0) {
    const bool masked = n0 + kTileKV - 1 > wave_first_pos || n0 + kTileKV > kvl || any_bad;
    f32x16 s0 = half_scores(buf, 0);
    f32x16 s1 = half_scores(buf, 1);
    rescale(half_max(s0, n0, 0, masked));
    V8 pb[2];
    probs(s0, pb);
    pv(buf, 0, pb);
    rescale(half_max(s1, n0, 1, masked));
    probs(s1, pb);
    pv(buf, 1, pb);
  };

  if constexpr (G::kLoadWaves > 0) {
    // Loader waves gather tile it + 1 into the LDS buffers tile it - 1 left
    // while the compute waves run tile it, and fetch tile it + 2 into their
    // one register set; one barrier per tile.
    const int t_first = kv_lo / kTileKV;
    if (wave >= G::kComputeWaves) {
      Regs ra;
      read_ids(kv_lo);
      fetch(ra);
      stash(0, ra);
      read_ids(kv_lo + kTileKV);
      fetch(ra);   // tile t_first + 1 (past the end: in-bounds reads, never stashed)
      read_ids(kv_lo + 2 * kTileKV);
      __syncthreads();   // tile t_first published
      for (int it = t_first; it < ntiles; ++it) {
        // Buffer (it + 1) % 2 was last read for tile it - 1, before the
        // previous barrier.
        if (it + 1 < ntiles) stash((it - t_first + 1) & 1, ra);
        fetch(ra);   // tile it + 2
        read_ids((it + 3) * kTileKV);
        __syncthreads();
      }
      return;
    }
    qf_load();
    __syncthreads();   // tile t_first published
    for (int it = t_first; it < ntiles; ++it) {
      const int n0 = it * kTileKV;
      if (wave_active && n0 <= wave_last_pos) compute((it - t_first) & 1, n0);
      __syncthreads();
    }
  } else {
  // Tile it is computed from LDS buffer it % 2 while tile it + 1 sits in
  // registers (loads issued one iteration earlier) and tile it + 2 is being
  // fetched into the other register set.
  qf_load();
  Regs ra, rb;
  read_ids(kv_lo);
  fetch(ra);
  read_ids(kv_lo + kTileKV);
  fetch(rb);
  stash(0, ra);
  read_ids(kv_lo + 2 * kTileKV);
  __syncthreads();
  for (int it = kv_lo / kTileKV; it < ntiles; it += 2) {
    // even tile: next tile in rb, fetch it + 2 into ra
    {
      const int n0 = it * kTileKV;
      fetch(ra);   // tile n0 + 2 (past the end: in-bounds reads, never stashed)
      if (wave_active && n0 <= wave_last_pos) compute(0, n0);
      if (it + 1 < ntiles) stash(1, rb);   // buffer 1 was last read before the previous barrier
      read_ids(n0 + 3 * kTileKV);
      __syncthreads();
    }
    if (it + 1 >= ntiles) break;
    // odd tile: next tile in ra, fetch it + 3 into rb
    {
      const int n0 = (it + 1) * kTileKV;
      fetch(rb);
      if (wave_active && n0 <= wave_last_pos) compute(1, n0);
      if (it + 2 < ntiles) stash(0, ra);
      read_ids(n0 + 3 * kTileKV);
      __syncthreads();
    }
  }
  }

  lsum += __shfl_xor(lsum, 32);
  if (!row_ok) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  if (slot < 0) {
    f16* op = a.out + int64_t(qt + qrow) * a.o_tok + int64_t(hq) * a.o_head;
#pragma unroll
    for (int dt = 0; dt < G::kBlocks; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const V4 val = {T(o[dt][4 * g] * inv), T(o[dt][4 * g + 1] * inv),
                        T(o[dt][4 * g + 2] * inv), T(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<V4*>(op + 32 * dt + 8 * g + 4 * h) = val;
      }
    return;
  }
  // Split: this KV range's normalised O, its running max and its sum. A row
  // that sees no key of the range has sum 0 (weight 0 in the merge).
  const int64_t prow = int64_t(slot) * G::kTileQ + (qrow - q0);
  float* po = a.part_o + prow * D;
#pragma unroll
  for (int dt = 0; dt < G::kBlocks; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 val = {o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                         o[dt][4 * g + 3] * inv};
      *reinterpret_cast<f32x4*>(po + 32 * dt + 8 * g + 4 * h) = val;
    }
  if (h == 0) {
    a.part_ml[2 * prow] = m;
    a.part_ml[2 * prow + 1] = lsum;
  }
}

// Warp-specialised variant for head_dim 64 and 128. A workgroup is 12
// waves: compute waves 0-7 (32 query rows each, two per SIMD) only read
// LDS and run the math; loader waves 8-11 (one per SIMD) only gather K/V
// tiles from the pages into LDS. Loaders run one tile ahead: with tiles
// counted from the item's first, tile u is written between barriers u - 2
// and u - 1, into K buffer u % 2 and V buffer u % 3, from registers loaded
// two tiles earlier. Compute waves run barrier t between the two 32-token
// halves of tile t (the second half's score MFMAs read K of tile t + 1,
// published by that barrier). The interior tiles, whose keys every row
// sees, run a straight-line pipeline (the scores of half-step j + 1 issue
// between the exponentials of j, and the P.V of j beside the max of j + 1);
// the diagonal tiles run each half on its own, with the causal /
// past-the-end / no-data masks. Waves with no row before q_len only pass
// the barriers.
template <int D>
struct WsGeom {
  static_assert(D == 64 || D == 128, "warp-specialised prefill is for head_dim 64 and 128");
  static constexpr int kComputeWaves = 8;
  static constexpr int kLoadWaves = 4;
  static constexpr int kWaves = kComputeWaves + kLoadWaves;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kTileQ = 32 * kComputeWaves;
  static constexpr int kSteps = D / 16;
  static constexpr int kBlocks = D / 32;
  static constexpr int kKPitch = D + 8;
  static constexpr int kKHalves = kTileKV * kKPitch;
  static constexpr int kVtHalves = D * kVtPitch;
  // Units (4 tokens x 8 dims of K or V) per loader lane: at 128 each loader
  // wave gathers V and K of one token group of 16 (the same lane layout for
  // both); at 64 loaders 0-1 gather V and 2-3 K, two token groups a wave.
  static constexpr int kUnits = D == 128 ? 2 : 1;
};

template <typename T, int D, bool STAGED>
__global__ __launch_bounds__(WsGeom<D>::kThreads) void paged_prefill_ws_kernel(PrefillArgs a) {
  typedef typename Vec<T>::v8 V8;
  typedef WsGeom<D> G;
  __shared__ int s_pg[STAGED ? kMaxStagedPages : 1];
  __shared__ int s_bad[G::kWaves];
  __shared__ __attribute__((aligned(16))) T sK[2 * G::kKHalves];
  __shared__ __attribute__((aligned(16))) T sVt[3 * G::kVtHalves];
  // Per K buffer, one byte per token of the tile: nonzero for a token with
  // no data (on a page outside the pool, or past the end of the range).
  __shared__ uint32_t s_inv[2][kTileKV / 4];

  const int32_t* item = a.tiles + kRec * blockIdx.x;
  const int seq = item[0];
  if (seq < 0) return;   // padding workgroup (uniform: no barrier reached)
  const int q0 = item[1];
  const int hq = item[2];
  const int kv_lo = item[3];   // a multiple of kTileKV
  const int kv_hi = item[4];
  const int slot = item[5];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = wave >= G::kComputeWaves;   // uniform per wave
  const int r = lane & 31;
  const int h = lane >> 5;

  const int hkv = hq / a.ratio;
  const int qb = a.q_indptr[seq];
  const int q_len = a.q_indptr[seq + 1] - qb;
  const int qt = a.q_start ? a.q_start[seq] : qb;   // the row's first token of q and out
  const int kvl = a.kv_len[seq];
  const int prefix = kvl - q_len;
  const int32_t* pages = a.indices + a.indptr[seq];
  const int page_mask = (1 << a.page_shift) - 1;
  const int kv_end = min(prefix + min(q0 + G::kTileQ, q_len), kv_hi);   // exclusive
  const int ntiles = (kv_end + kTileKV - 1) / kTileKV;   // tiles [kv_lo / kTileKV, ntiles)
  const int t_first = kv_lo / kTileKV;
  const int pg_lo = kv_lo >> a.page_shift;

  // Loader lanes: gather layout, tile registers, position lookups.
  const int lw = wave - G::kComputeWaves;
  const GatherLane gl = gather_lane<D>(D == 128 ? lw : lw % 2, lane);
  const int ld_t = 16 * gl.g + 8 * gl.a + 4 * gl.h;
  auto unit_v = [&](int u) { return D == 128 ? u == 0 : lw < 2; };
  const f16* kbase = a.k + int64_t(hkv) * a.head_stride;
  const f16* vbase = a.v + int64_t(hkv) * a.head_stride;
  struct Regs {
    V8 x[G::kUnits][4];
    int nok;
  };
  TileAt at;
  auto read_ids = [&](int n0) {
    const int tok = n0 + ld_t;
    const int t = max(kv_lo, min(tok, kv_end - 1));   // clamped into the staged range
    const int p = STAGED ? s_pg[(t >> a.page_shift) - pg_lo] : pages[t >> a.page_shift];
    at = tile_at(p, tok, kv_end, a.num_pages, a.page_stride, a.token_stride, page_mask, 8 * gl.c);
  };
  auto read_ids_global = [&](int n0) {
    const int tok = n0 + ld_t;
    const int t = max(kv_lo, min(tok, kv_end - 1));
    at = tile_at(pages[t >> a.page_shift], tok, kv_end, a.num_pages, a.page_stride, a.token_stride,
                 page_mask, 8 * gl.c);
  };
  auto fetch = [&](Regs& rg) {
#pragma unroll
    for (int u = 0; u < G::kUnits; ++u) {
      const f16* base = (unit_v(u) ? vbase : kbase) + at.off;
#pragma unroll
      for (int i = 0; i < 4; ++i) rg.x[u][i] = load_v8<T>(base + int64_t(i) * a.token_stride);
    }
    rg.nok = at.nok;
  };
  auto stash = [&](int kbuf, int vbuf, const Regs& rg) {
#pragma unroll
    for (int u = 0; u < G::kUnits; ++u) {
      if (unit_v(u)) {
#pragma unroll
        for (int part = 0; part < 4; ++part)
          vt_store<T>(sVt + vbuf * G::kVtHalves, gl, gl.c, rg.x[u], part, rg.nok);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<V8*>(&sK[kbuf * G::kKHalves + (ld_t + i) * G::kKPitch + 8 * gl.c]) =
              rg.x[u][i];
        // The K lanes of chunk 0 flag their 4 tokens (byte i: token i has no data).
        if (gl.c == 0)
          s_inv[kbuf][ld_t / 4] = rg.nok >= 4 ? 0u : 0x01010101u << (8 * rg.nok);
      }
    }
  };
  // Row block of a compute wave: waves w and w + 4 share a SIMD, and take
  // blocks w and 7 - w, so that each SIMD pairs a short and a long run of
  // diagonal half-steps (block b sees keys up to its own rows).
  const int blk = wave < 4 ? wave : 11 - wave;
  const int qrow = q0 + blk * 32 + r;
  const bool row_ok = qrow < q_len;
  const int npg = kv_end > kv_lo ? ((kv_end - 1) >> a.page_shift) + 1 - pg_lo : 0;
  if (loader) {
    // ---------------------------------------------------------- loader
    // Tile t_first + k is in register set k % 2 (ra even, rb odd). The
    // barrier after iteration u is barrier u - 1 of the compute waves.
    // The first two tiles' loads go out while the compute waves stage the
    // page ids, with their ids read from the table directly.
    Regs ra, rb;
    read_ids_global(kv_lo);
    fetch(ra);
    read_ids_global(kv_lo + kTileKV);
    fetch(rb);
    __syncthreads();   // page ids staged
    stash(0, 0, ra);
    read_ids(kv_lo + 2 * kTileKV);
    fetch(ra);   // tile t_first + 2 (past the end: in-bounds reads, never stashed)
    read_ids(kv_lo + 3 * kTileKV);
    __syncthreads();
    int kb = 1, vbn = 1;   // buffers of tile t_first + 1
    auto advance = [&]() {
      kb ^= 1;
      vbn = vbn == 2 ? 0 : vbn + 1;
    };
    for (int u = t_first + 1; u <= ntiles; u += 2) {
      if (u < ntiles) stash(kb, vbn, rb);
      fetch(rb);   // tile u + 2
      read_ids((u + 3) * kTileKV);
      __syncthreads();
      advance();
      if (u + 1 > ntiles) break;
      if (u + 1 < ntiles) stash(kb, vbn, ra);
      fetch(ra);   // tile u + 3
      read_ids((u + 4) * kTileKV);
      __syncthreads();
      advance();
    }
    return;
  }

  // ------------------------------------------------------------ compute
  // Stage (or, for rows with too many pages, only scan) the page ids of
  // [kv_lo, kv_end) and vote whether any is outside the pool.
  bool any_bad = false;
  {
    bool bad_id = false;
    for (int i = threadIdx.x; i < npg; i += G::kComputeWaves * kWave) {
      const int p = pages[pg_lo + i];
      const bool ok = p >= 0 && p < a.num_pages;
      if constexpr (STAGED) s_pg[i] = ok ? p : -1;
      bad_id |= !ok;
    }
    const bool wave_bad = __any(bad_id);
    if (lane == 0) s_bad[wave] = wave_bad;
    __syncthreads();   // page ids staged
    int bad = 0;
#pragma unroll
    for (int wv = 0; wv < G::kComputeWaves; ++wv) bad |= s_bad[wv];
    any_bad = __builtin_amdgcn_readfirstlane(bad) != 0;
  }
  // Q as the B operand of S^T = K.Q^T: step s covers dims 16s + 8h .. +8
  // (a row past q_len reads the sequence's first row and writes nothing).
  V8 qf[G::kSteps];
  {
    const f16* qp = a.q + int64_t(qt + (row_ok ? qrow : 0)) * a.q_tok + int64_t(hq) * a.q_head;
#pragma unroll
    for (int s = 0; s < G::kSteps; ++s) qf[s] = load_v8<T>(qp + 16 * s + 8 * h);
  }
  const int qpos = prefix + qrow;
  f32x16 o[G::kBlocks];
#pragma unroll
  for (int i = 0; i < G::kBlocks; ++i) o[i] = f32x16{};
  float m = -1.0e30f;   // running max of this row, in log2 units
  float lsum = 0.f;     // this lane's share of the row sum (other half: lane ^ 32)
  V8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = T(1.f);

  const int kb0 = r * G::kKPitch + 8 * h;
  const VtBases vb = vt_operand_bases(lane);
  // Half-step j covers kv tokens [32 j, 32 j + 32): K rows 32 (j % 2) ..
  // of its tile's K buffer, V^T k-steps 2 (j % 2), 2 (j % 2) + 1. Lane
  // (r, h) holds tokens 32 j + 8 (v / 4) + 4 h + v % 4 of row r.
  auto half_scores = [&](int kbuf, int hh) {
    const T* kt = sK + kbuf * G::kKHalves + kb0 + 32 * hh * G::kKPitch;
    f32x16 s = mfma32(*reinterpret_cast<const V8*>(kt), qf[0], f32x16{});
#pragma unroll
    for (int st = 1; st < G::kSteps; ++st)
      s = mfma32(*reinterpret_cast<const V8*>(kt + 16 * st), qf[st], s);
    return s;
  };
  // Row max in log2 units (lanes r and r + 32 hold the two halves of row r).
  auto row_max = [&](const f32x16& s) {
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
    const auto sw = __builtin_amdgcn_permlane32_swap(f32_to_bits(mx), f32_to_bits(mx), false, false);
    return fmaxf(bits_to_f32(sw[0]), bits_to_f32(sw[1])) * a.scale_log2;
  };
  // Lazy running max: moved only when a row's max exceeds it by more than
  // 8 (log2 units), so probabilities stay <= 2^8 (far inside the fp16
  // range), and the O rescale is skipped unless some row of the wave moved.
  auto rescale = [&](float mx) {
    if (__any(mx > m + 8.f)) {
      const float m_new = mx > m + 8.f ? mx : m;
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < G::kBlocks; ++dt) o[dt] *= alpha;
    }
  };
  // P^T operands: k-step kk covers tokens 16 kk + 4 h + {0..3} and
  // 16 kk + 8 + 4 h + {0..3}, i.e. score entries 8 kk + e. The row sum is
  // taken over the rounded probabilities the P.V product uses.
  auto probs = [&](const f32x16& s, V8 (&pb)[2]) {
#pragma unroll
    for (int v = 0; v < 16; ++v) pb[v >> 3][v & 7] = T(fast_exp2(fmaf(s[v], a.scale_log2, -m)));
    lsum = dot8(pb[0], ones, lsum);
    lsum = dot8(pb[1], ones, lsum);
  };
  auto pv = [&](int vbuf, int hh, const V8 (&pb)[2]) {
    const T* vt = sVt + vbuf * G::kVtHalves;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ks = 2 * hh + kk;
#pragma unroll
      for (int dt = 0; dt < G::kBlocks; ++dt) {
        const V8 va = *reinterpret_cast<const V8*>(vt + vb.b[vt_operand_base_index(ks, dt)] +
                                                    vt_operand_offset(dt));
        o[dt] = mfma32(va, pb[kk], o[dt]);
      }
    }
  };

  // Interior tiles [t_first, t_int): before the workgroup's first row, in
  // the KV range, no page id outside the pool.
  const int t_int = any_bad ? t_first : max(t_first, min(ntiles, (prefix + q0 + 1) / kTileKV));
  f32x16 sc;   // scores of the current half-step
  // Pipelined step: V of the current half-step in V buffer vbuf (half hh),
  // K of the next in K buffer kbuf_n (half hh_n).
  auto step = [&](int kbuf_n, int hh_n, int vbuf, int hh) {
    V8 pb[2];
    const f32x16 sn = half_scores(kbuf_n, hh_n);
    probs(sc, pb);
    pv(vbuf, hh, pb);
    const float mx = row_max(sn);
    sc = sn;
    rescale(mx);
  };
  auto step_last = [&](int vbuf, int hh) {
    V8 pb[2];
    probs(sc, pb);
    pv(vbuf, hh, pb);
  };
  // Masks of half-step j's scores: causal and past the end of the row
  // (tokens >= min(qpos + 1, kvl)), and tokens the loaders flagged as having
  // no data. Lane (r, h) entry 4 v4 + e is token 32 j + 8 v4 + e + 4 h.
  const int lim0 = min(qpos + 1, kvl);
  auto mask = [&](f32x16& sv, int j, int kbuf) {
    // The bound is made opaque so that the compiler compares it with the
    // 16 immediates instead of keeping 16 precomputed bounds live.
    int lim = lim0 - 32 * j - 4 * h;
    asm volatile("" : "+v"(lim));
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      // The loaders' flags of the group's 4 tokens.
      const uint32_t inv = s_inv[kbuf][8 * (j & 1) + 2 * v4 + h];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (((inv >> (8 * e)) & 1) || 8 * v4 + e >= lim) sv[4 * v4 + e] = -INFINITY;
    }
  };
  // Diagonal tiles: a wave runs the half-steps up to its last visible key.
  const bool wave_active = q0 + blk * 32 < q_len;
  const int wave_last_pos = prefix + min(q0 + blk * 32 + 31, q_len - 1);
  const int j_last = wave_active ? min(wave_last_pos, kv_end - 1) >> 5 : -1;
  auto half_masked = [&](int kbuf, int vbuf, int j) {
    if (j > j_last) return;   // uniform per wave
    f32x16 sv = half_scores(kbuf, j & 1);
    mask(sv, j, kbuf);
    rescale(row_max(sv));
    V8 pb[2];
    probs(sv, pb);
    pv(vbuf, j & 1, pb);
  };

  __syncthreads();   // tile t_first published
  int kcur = 0, vcur = 0;
  auto tile_end = [&]() {
    kcur ^= 1;
    vcur = vcur == 2 ? 0 : vcur + 1;
  };
  // Interior tiles: every wave with a row before q_len runs pipelined plain
  // steps (its rows past q_len on the first row's q).
  if (!wave_active) {
    // Every row of this wave is past q_len: only the barriers.
    for (int it = t_first; it < t_int; ++it) {
      __syncthreads();
      tile_end();
    }
  } else if (t_int > t_first) {
    sc = half_scores(0, 0);
    rescale(row_max(sc));
    for (int it = t_first; it + 1 < t_int; ++it) {
      step(kcur, 1, vcur, 0);
      __syncthreads();
      step(kcur ^ 1, 0, vcur, 1);
      tile_end();
    }
    step(kcur, 1, vcur, 0);
    __syncthreads();
    step_last(vcur, 1);
    tile_end();
  }
  // The wave's rows are final after its last visible key: writes them
  // (normalised, or as split partials).
  auto finish = [&]() {
    lsum += __shfl_xor(lsum, 32);
    if (!row_ok) return;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    if (slot < 0) {
      typedef typename Vec<T>::v4 V4;
      f16* op = a.out + int64_t(qt + qrow) * a.o_tok + int64_t(hq) * a.o_head;
#pragma unroll
      for (int dt = 0; dt < G::kBlocks; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const V4 val = {T(o[dt][4 * g] * inv), T(o[dt][4 * g + 1] * inv),
                          T(o[dt][4 * g + 2] * inv), T(o[dt][4 * g + 3] * inv)};
          *reinterpret_cast<V4*>(op + 32 * dt + 8 * g + 4 * h) = val;
        }
      return;
    }
    const int64_t prow = int64_t(slot) * G::kTileQ + (qrow - q0);
    float* po = a.part_o + prow * D;
#pragma unroll
    for (int dt = 0; dt < G::kBlocks; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 val = {o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                           o[dt][4 * g + 3] * inv};
        *reinterpret_cast<f32x4*>(po + 32 * dt + 8 * g + 4 * h) = val;
      }
    if (h == 0) {
      a.part_ml[2 * prow] = m;
      a.part_ml[2 * prow + 1] = lsum;
    }
  };
  // Diagonal tiles. A wave writes its rows right after the tile of its last
  // visible key, before that tile's barrier, and then only passes the
  // remaining barriers: its stores drain while the waves with more diagonal
  // half-steps (rows further down) still compute. Writing every wave's rows
  // after the last barrier left a workgroup's output (64 KiB at head_dim
  // 128) to drain with its CU otherwise idle, about 4% of the chunked-prefill
  // workload's time.
  const int it_last = min(ntiles - 1, j_last >> 1);   // uniform; < t_int: no visible key here
  int it = t_int;
  for (; it < it_last; ++it) {
    half_masked(kcur, vcur, 2 * it);
    half_masked(kcur, vcur, 2 * it + 1);
    __syncthreads();
    tile_end();
  }
  if (it == it_last) {
    half_masked(kcur, vcur, 2 * it);
    half_masked(kcur, vcur, 2 * it + 1);
  }
  finish();
  for (; it < ntiles; ++it) {   // the barrier of tile it_last, then those of the later tiles
    __syncthreads();
    tile_end();
  }
}

// Combines the splits of one (sequence, q tile, q head): weight of split j
// = 2^(m_j - max m) * sum_j, taken in split order.
struct MergeArgs {
  const int32_t* merges;   // [num_merge][kMergeRec]
  const float* part_o;
  const float* part_ml;
  const int32_t* q_indptr;
  const int32_t* q_start;  // as PrefillArgs::q_start
  f16* out;
  int64_t o_tok, o_head;
};

// Grid (merge record, block of merge_rows(D) rows); one thread per (row, 8 dims).
constexpr int merge_rows(int head_dim) { return 256 / (head_dim / 8); }

template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(MergeArgs a) {
  typedef typename Vec<T>::v4 V4;
  constexpr int kTileQ = Geom<D>::kTileQ;
  const int32_t* rec = a.merges + kMergeRec * blockIdx.x;
  const int seq = rec[0], q0 = rec[1], hq = rec[2], s0 = rec[3], n = rec[4];
  const int qb = a.q_indptr[seq];
  const int q_len = a.q_indptr[seq + 1] - qb;
  const int qt = a.q_start ? a.q_start[seq] : qb;   // the row's first token of q and out
  {
    const int row = blockIdx.y * merge_rows(D) + int(threadIdx.x) / (D / 8);
    const int c = int(threadIdx.x) % (D / 8);
    if (q0 + row >= q_len) return;
    // Splits are read 8 at a time, each batch's loads issued together: one
    // split at a time would wait a memory round trip per split (12 us
    // against 9 us for an 8-way split of 32 tiles of 216 rows).
    constexpr int kBatch = 8;
    float mx = -INFINITY;
    for (int j0 = 0; j0 < n; j0 += kBatch) {
      float mm[kBatch], ll[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t pr = int64_t(s0 + j0 + u) * kTileQ + row;
        const bool in = j0 + u < n;
        mm[u] = in ? a.part_ml[2 * pr] : -INFINITY;
        ll[u] = in ? a.part_ml[2 * pr + 1] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (ll[u] > 0.f) mx = fmaxf(mx, mm[u]);
    }
    float wsum = 0.f, acc[8] = {};
    for (int j0 = 0; j0 < n; j0 += kBatch) {
      float mm[kBatch], ll[kBatch];
      f32x4 x0[kBatch], x1[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t pr = int64_t(s0 + j0 + u) * kTileQ + row;
        const bool in = j0 + u < n;
        mm[u] = in ? a.part_ml[2 * pr] : 0.f;
        ll[u] = in ? a.part_ml[2 * pr + 1] : 0.f;
        x0[u] = in ? *reinterpret_cast<const f32x4*>(a.part_o + pr * D + 8 * c) : f32x4{};
        x1[u] = in ? *reinterpret_cast<const f32x4*>(a.part_o + pr * D + 8 * c + 4) : f32x4{};
      }
      // in split order, so the result does not depend on timing
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (!(ll[u] > 0.f)) continue;
        const float w = fast_exp2(mm[u] - mx) * ll[u];
        wsum += w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] = fmaf(w, x0[u][e], acc[e]);
          acc[4 + e] = fmaf(w, x1[u][e], acc[4 + e]);
        }
      }
    }
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
    f16* op = a.out + int64_t(qt + q0 + row) * a.o_tok + int64_t(hq) * a.o_head + 8 * c;
    *reinterpret_cast<V4*>(op) = {T(acc[0] * inv), T(acc[1] * inv), T(acc[2] * inv),
                                  T(acc[3] * inv)};
    *reinterpret_cast<V4*>(op + 4) = {T(acc[4] * inv), T(acc[5] * inv), T(acc[6] * inv),
                                      T(acc[7] * inv)};
  }
}

// ------------------------------------------------------------ append

// Step tokens per append workgroup. The workgroup resolves its tokens'
// rows, positions and page slots once, into LDS, and then streams their
// heads: a head's 16 tokens are consecutive slots of one page (two when the
// tile straddles a page boundary), so its stores form 4 KiB runs at
// head_dim 128. The new k and v are read with non-temporal loads (streamed
// once): on the chunked-prefill workload they measured 4.9 TB/s against
// 4.2 TB/s with plain loads.
constexpr int kAppendTok = 16;
constexpr int kAppendThreads = 256;

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
};

// Position of step token `tok` in its row b (the largest b with
// q_indptr[b] <= tok): kv_len[b] - q_len[b] + (tok - q_indptr[b]), or -1
// for a token no row owns or a position outside [0, kv_len[b]). `slot` is
// the element offset of the position's page slot in the layer (page *
// page_stride + slot * token_stride), or -1 when the page id is outside
// the pool.
__device__ __forceinline__ int token_position(const AppendArgs& a, int tok, int64_t& slot) {
  slot = -1;
  if (tok >= a.num_tokens || tok >= a.q_indptr[a.num_seqs] || tok < a.q_indptr[0]) return -1;
  int lo = 0, hi = a.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.q_indptr[mid] <= tok) lo = mid; else hi = mid - 1;
  }
  const int qb = a.q_indptr[lo];
  const int kvl = a.kv_len[lo];
  const int pos = kvl - (a.q_indptr[lo + 1] - qb) + (tok - qb);
  if (pos < 0 || pos >= kvl) return -1;
  const int p = a.indices[a.indptr[lo] + (pos >> a.page_shift)];
  if (p >= 0 && p < a.num_pages)
    slot = int64_t(p) * a.page_stride + int64_t(pos & ((1 << a.page_shift) - 1)) * a.token_stride;
  return pos;
}

// token_position of tokens tok0 + lane for lanes < TT, run by one whole
// wave (every lane calls it; lanes >= TT get -1). With fewer
// than 64 rows the wave loads q_indptr once and finds each token's row by
// counting the row starts at or before it (a ballot), so the lookup costs
// three dependent memory round trips (q_indptr; kv_len and indptr; the page
// id) instead of a binary search's log2(rows) more.
template <int TT>
__device__ __forceinline__ int tile_positions(const AppendArgs& a, int tok0, int64_t& slot) {
  const int lane = int(threadIdx.x) % kWave;
  const int tok = tok0 + lane;
  slot = -1;
  const int ns = a.num_seqs;
  if (ns >= kWave) return lane < TT ? token_position(a, tok, slot) : -1;
  const int qi = a.q_indptr[lane < ns ? lane : ns];
  int b = 0;
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const uint64_t m = __ballot(lane >= 1 && lane < ns && qi <= tok0 + t);
    if (lane == t) b = __popcll(m);
  }
  const int qb = __shfl(qi, b), qe = __shfl(qi, b + 1);
  const int first = __shfl(qi, 0), total = __shfl(qi, ns);
  if (lane >= TT || tok >= a.num_tokens || tok >= total || tok < first) return -1;
  const int kvl = a.kv_len[b];
  const int pos = kvl - (qe - qb) + (tok - qb);
  if (pos < 0 || pos >= kvl) return -1;
  const int p = a.indices[a.indptr[b] + (pos >> a.page_shift)];
  if (p >= 0 && p < a.num_pages)
    slot = int64_t(p) * a.page_stride + int64_t(pos & ((1 << a.page_shift) - 1)) * a.token_stride;
  return pos;
}

// Workgroup = kAppendTok step tokens x 128 / CPR KV heads (CPR = head_dim /
// 8 sixteen-byte chunks per head row): every thread keeps one (head, chunk)
// and moves it for 8 of the tokens, K and V. Waves 1-3 issue their 16 loads
// at once, so their latency overlaps wave 0's row search.
template <int CPR>
__global__ __launch_bounds__(kAppendThreads) void append_kv_kernel(AppendArgs a) {
  constexpr int kHeads = 128 / CPR;
  constexpr int kIters = kAppendTok * 128 / kAppendThreads;   // 8 tokens per thread
  __shared__ int64_t s_slot[kAppendTok];
  const int tok0 = int(blockIdx.x) * kAppendTok;
  const int head = int(blockIdx.y) * kHeads + int(threadIdx.x & 127) / CPR;
  const int c = int(threadIdx.x) % CPR;
  const int t_first = int(threadIdx.x) >> 7;   // tokens t_first, t_first + 2, ...
  const bool head_ok = head < a.num_kv_heads;
  // Wave 0 resolves the tile's slots before it issues its own loads: the
  // memory counter waits in issue order, so a lookup issued after the data
  // loads would wait for all of them.
  if (threadIdx.x < kWave) {
    int64_t slot;
    const int pos = tile_positions<kAppendTok>(a, tok0, slot);
    if (threadIdx.x < kAppendTok) s_slot[threadIdx.x] = pos >= 0 ? slot : int64_t(-1);
  }
  f16x8 kx[kIters], vx[kIters];
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const int tok = tok0 + t_first + 2 * i;
    if (head_ok && tok < a.num_tokens) {
      kx[i] = load_f16x8_nt(a.k_new + int64_t(tok) * a.k_tok + int64_t(head) * a.k_head + c * 8);
      vx[i] = load_f16x8_nt(a.v_new + int64_t(tok) * a.v_tok + int64_t(head) * a.v_head + c * 8);
    }
  }
  __syncthreads();
  if (!head_ok) return;
  const int64_t hc = int64_t(head) * a.head_stride + c * 8;
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const int64_t slot = s_slot[t_first + 2 * i];
    if (slot >= 0) {
      store_f16x8(a.k + slot + hc, kx[i]);
      store_f16x8(a.v + slot + hc, vx[i]);
    }
  }
}

// Fused prologue of a step: rotary position embedding of q (in place) and
// of the new k, and the append of the rotated k and of v into the pages.
// One workgroup per token: its D/2 rotation angles are evaluated once
// (fp32 product position * inv_freq[j], accurate sincosf) into LDS, then
// the workgroup streams the token's heads in units of 16 dims: units of
// head slots [0, Hq) are q heads (rotated in place), of [Hq, Hq + Hkv) KV
// heads (k rotated and written, the same dims of v copied). Rotation pairs
// are (j, j + D/2) with a unit's dims 8c..8c+7 and D/2 + 8c..+7, or
// (2j, 2j + 1) with dims 16c..16c+15 when interleaved. fp32 rotation, one
// rounding.
struct RopeArgs {
  f16* q;
  int64_t q_tok, q_head;
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
  const float* inv_freq;   // [D / 2]
  int32_t num_seqs;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t interleave;
};

__device__ __forceinline__ void rope_pair(float& a, float& b, float c, float s) {
  const float x = a, y = b;
  a = fmaf(x, c, -y * s);
  b = fmaf(y, c, x * s);
}

constexpr int kRopeThreads = 256;

template <typename T>
__global__ __launch_bounds__(kRopeThreads) void rope_append_kernel(RopeArgs a) {
  typedef typename Vec<T>::v8 V8;
  __shared__ float s_cos[128], s_sin[128];   // head_dim <= 256
  const int tok = blockIdx.x;
  if (tok >= a.q_indptr[a.num_seqs]) return;   // not owned by any row (uniform)
  int lo = 0, hi = a.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.q_indptr[mid] <= tok) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int q_len = a.q_indptr[b + 1] - a.q_indptr[b];
  const int pos = a.kv_len[b] - q_len + (tok - a.q_indptr[b]);
  if (pos < 0 || pos >= a.kv_len[b]) return;   // uniform
  const int half = a.head_dim / 2;
  for (int j = threadIdx.x; j < half; j += kRopeThreads)
    sincosf(float(pos) * a.inv_freq[j], &s_sin[j], &s_cos[j]);
  __syncthreads();

  const int p = a.indices[a.indptr[b] + (pos >> a.page_shift)];
  const bool page_ok = p >= 0 && p < a.num_pages;
  const int64_t dst = int64_t(page_ok ? p : 0) * a.page_stride +
                      int64_t(pos & ((1 << a.page_shift) - 1)) * a.token_stride;
  const int units = a.head_dim / 16;
  const int n_units = (a.num_qo_heads + a.num_kv_heads) * units;
  for (int u = threadIdx.x; u < n_units; u += kRopeThreads) {
    const int slot = u / units, c = u % units;
    const int d0 = a.interleave ? 16 * c : 8 * c;
    const int d1 = a.interleave ? 16 * c + 8 : half + 8 * c;
    auto rotate = [&](const V8& x0, const V8& x1, V8& y0, V8& y1) {
      float w[16];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        w[e] = float(x0[e]);
        w[8 + e] = float(x1[e]);
      }
      if (a.interleave) {
        // dims 16c + 2j, 16c + 2j + 1 hold pair 8c + j
#pragma unroll
        for (int j = 0; j < 8; ++j) rope_pair(w[2 * j], w[2 * j + 1], s_cos[8 * c + j], s_sin[8 * c + j]);
      } else {
        // dims 8c + j and D/2 + 8c + j hold pair 8c + j
#pragma unroll
        for (int j = 0; j < 8; ++j) rope_pair(w[j], w[8 + j], s_cos[8 * c + j], s_sin[8 * c + j]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y0[e] = T(w[e]);
        y1[e] = T(w[8 + e]);
      }
    };
    V8 y0, y1;
    if (slot < a.num_qo_heads) {
      f16* qp = a.q + int64_t(tok) * a.q_tok + int64_t(slot) * a.q_head;
      rotate(load_v8<T>(qp + d0), load_v8<T>(qp + d1), y0, y1);
      *reinterpret_cast<V8*>(qp + d0) = y0;
      *reinterpret_cast<V8*>(qp + d1) = y1;
      continue;
    }
    if (!page_ok) continue;
    const int head = slot - a.num_qo_heads;
    const int64_t hd = dst + int64_t(head) * a.head_stride;
    const f16* kp = a.k_new + int64_t(tok) * a.k_tok + int64_t(head) * a.k_head;
    const f16* vp = a.v_new + int64_t(tok) * a.v_tok + int64_t(head) * a.v_head;
    rotate(load_v8<T>(kp + d0), load_v8<T>(kp + d1), y0, y1);
    *reinterpret_cast<V8*>(a.k + hd + d0) = y0;
    *reinterpret_cast<V8*>(a.k + hd + d1) = y1;
    store_f16x8(a.v + hd + d0, load_f16x8(vp + d0));
    store_f16x8(a.v + hd + d1, load_f16x8(vp + d1));
  }
}

// Attention (page ids staged in LDS when they fit), then the split merge.
template <typename T, int D>
int run_prefill(const PrefillArgs& a, const MergeArgs& m, int num_tiles, int num_merge,
                bool staged, hipStream_t s) {
  if constexpr (D <= 128) {
    constexpr int kThreads = WsGeom<D>::kThreads;
    if (staged)
      paged_prefill_ws_kernel<T, D, true><<<dim3(num_tiles), kThreads, 0, s>>>(a);
    else
      paged_prefill_ws_kernel<T, D, false><<<dim3(num_tiles), kThreads, 0, s>>>(a);
  } else {
    constexpr int kThreads = Geom<D>::kThreads;
    if (staged)
      paged_prefill_kernel<T, D, true><<<dim3(num_tiles), kThreads, 0, s>>>(a);
    else
      paged_prefill_kernel<T, D, false><<<dim3(num_tiles), kThreads, 0, s>>>(a);
  }
  KSV_CHECK_LAUNCH();
  if (num_merge > 0) {
    prefill_merge_kernel<T, D><<<dim3(num_merge, Geom<D>::kTileQ / merge_rows(D)), 256, 0, s>>>(m);
    KSV_CHECK_LAUNCH();
  }
  return KUNSERVE_OK;
}

template <typename T>
int run_prefill_dim(int head_dim, const PrefillArgs& a, const MergeArgs& m, int num_tiles,
                    int num_merge, bool staged, hipStream_t s) {
  switch (head_dim) {
    case 64: return run_prefill<T, 64>(a, m, num_tiles, num_merge, staged, s);
    case 128: return run_prefill<T, 128>(a, m, num_tiles, num_merge, staged, s);
    default: return run_prefill<T, 256>(a, m, num_tiles, num_merge, staged, s);
  }
}

}  // namespace
}  // namespace kunserve

using namespace kunserve;

extern "C" int kunserve_rope_append_kv(const kunserve_kv_pool* pool, int32_t layer,
                                       const kunserve_page_table* table,
                                       const int32_t* q_indptr_dev, int32_t num_tokens,
                                       kunserve_tensor3* q, int32_t num_qo_heads,
                                       const kunserve_tensor3* k_new,
                                       const kunserve_tensor3* v_new, const float* inv_freq_dev,
                                       int32_t interleave, kunserve_stream_t stream) {
  clear_error();
  int rc = check_pool(pool, true);
  if (rc) return rc;
  KSV_CHECK_ARG(table && q && k_new && v_new, "null argument");
  KSV_CHECK_ARG(layer >= 0 && layer < pool->num_layers, "layer %d outside [0, %d)", layer,
                pool->num_layers);
  KSV_CHECK_ARG(num_tokens >= 0, "num_tokens < 0");
  KSV_CHECK_ARG(num_qo_heads > 0 && num_qo_heads % pool->num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads,
                pool->num_kv_heads);
  KSV_CHECK_ARG(pool->head_dim % 16 == 0, "head_dim %d is not a multiple of 16", pool->head_dim);
  if (num_tokens == 0 || table->num_seqs == 0) return KUNSERVE_OK;
  KSV_CHECK_ARG(q_indptr_dev && table->indptr_dev && table->indices_dev && table->kv_len_dev &&
                    inv_freq_dev,
                "null table array or inv_freq");
  for (const kunserve_tensor3* t : {static_cast<const kunserve_tensor3*>(q), k_new, v_new})
    KSV_CHECK_ARG(t->data && aligned16(t->data) && t->token_stride % 8 == 0 &&
                      t->head_stride % 8 == 0,
                  "q / k_new / v_new must be 16-byte aligned with strides that are multiples of 8");
  RopeArgs a{};
  a.q = static_cast<f16*>(q->data);
  a.q_tok = q->token_stride;
  a.q_head = q->head_stride;
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
  a.inv_freq = inv_freq_dev;
  a.num_seqs = table->num_seqs;
  a.num_qo_heads = num_qo_heads;
  a.num_kv_heads = pool->num_kv_heads;
  a.head_dim = pool->head_dim;
  a.interleave = interleave != 0;
  // One workgroup per token.
  if (pool->dtype == KUNSERVE_DTYPE_BF16)
    rope_append_kernel<bf16><<<dim3(unsigned(num_tokens)), kRopeThreads, 0,
                               reinterpret_cast<hipStream_t>(stream)>>>(a);
  else
    rope_append_kernel<f16><<<dim3(unsigned(num_tokens)), kRopeThreads, 0,
                              reinterpret_cast<hipStream_t>(stream)>>>(a);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

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
  const int heads_per_wg = 128 / (pool->head_dim / 8);
  const dim3 grid(unsigned((num_tokens + kAppendTok - 1) / kAppendTok),
                  unsigned((pool->num_kv_heads + heads_per_wg - 1) / heads_per_wg));
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (pool->head_dim) {
    case 64: append_kv_kernel<8><<<grid, kAppendThreads, 0, s>>>(a); break;
    case 128: append_kv_kernel<16><<<grid, kAppendThreads, 0, s>>>(a); break;
    default: append_kv_kernel<32><<<grid, kAppendThreads, 0, s>>>(a); break;
  }
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}

// Splits: a step with fewer q-tile workgroups than CUs splits the KV range
// of its tiles into about kSplitWaves workgroups per CU, each covering at
// least kMinSplitTiles KV tiles (a multiple of kTileKV). One: at head_dim
// 128 a CU holds one workgroup at a time (76 KiB of LDS, 512 threads), so
// the splits run in a single round (measured on the chunked-prefill
// workload's last step: 0.047 ms, against 0.065 ms with two per CU and
// 0.077 ms with three).
constexpr int kSplitWaves = 1;
constexpr int kMinSplitTiles = 4;
constexpr int kMaxSplitItems = 2 * 1024;   // upper bound of the split target

static bool prefill_head_dim_ok(int32_t head_dim) {
  return head_dim == 64 || head_dim == 128 || head_dim == 256;
}

extern "C" int64_t kunserve_prefill_plan_bound(const int32_t* q_indptr_host, int32_t num_seqs,
                                               int32_t num_qo_heads, int32_t head_dim) {
  if (num_seqs < 0 || num_qo_heads <= 0 || (num_seqs > 0 && !q_indptr_host) ||
      !prefill_head_dim_ok(head_dim))
    return -1;
  const int32_t tile_q = tile_q_for(head_dim);
  int64_t tiles = 0;
  for (int32_t b = 0; b < num_seqs; ++b)
    tiles += (std::max(q_indptr_host[b + 1] - q_indptr_host[b], 0) + tile_q - 1) / tile_q;
  const int64_t items = tiles * num_qo_heads;
  // Splitting adds at most kMaxSplitItems workgroups; worst case every item
  // on one XCD and the others padded to the same depth; one merge record per
  // item.
  return int64_t(kRec) * kXcds * (items + kMaxSplitItems + 1) + int64_t(kMergeRec) * items;
}

extern "C" int kunserve_prefill_plan(const int32_t* q_indptr_host, const int32_t* kv_len_host,
                                     int32_t num_seqs, int32_t num_qo_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t num_cus,
                                     int32_t* plan_host, int64_t plan_capacity,
                                     kunserve_prefill_plan_info* info) {
  clear_error();
  KSV_CHECK_ARG(info && plan_host && num_seqs >= 0, "bad argument");
  if (!prefill_head_dim_ok(head_dim)) {
    set_error("prefill supports head_dim 64, 128 and 256, got %d", head_dim);
    return KUNSERVE_EUNSUPPORTED;
  }
  const int32_t tile_q = tile_q_for(head_dim);
  KSV_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads, num_kv_heads);
  KSV_CHECK_ARG(num_cus >= 0, "num_cus %d < 0", num_cus);
  if (num_seqs > 0) KSV_CHECK_ARG(q_indptr_host && kv_len_host, "null q_indptr / kv_len");
  const int ratio = num_qo_heads / num_kv_heads;
  // A group = (sequence, KV head, q-tile range): its items (all `ratio` q
  // heads of each tile) read the same K/V. Groups go to XCDs greedily, most
  // work first. A (sequence, KV head) keeps all its tiles in one group
  // unless there are too few groups to spread over the XCDs.
  struct Group { int32_t seq, hkv, t0, t1; int64_t cost; };
  int64_t n_pairs = 0, n_items = 0, kv_units = 0;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t ql = q_indptr_host[b + 1] - q_indptr_host[b];
    KSV_CHECK_ARG(ql >= 0, "q_indptr not monotone at %d", b);
    KSV_CHECK_ARG(kv_len_host[b] >= ql, "kv_len[%d] = %d < q_len %d", b, kv_len_host[b], ql);
    if (ql == 0) continue;
    n_pairs += num_kv_heads;
    const int32_t prefix = kv_len_host[b] - ql;
    for (int32_t q0 = 0; q0 < ql; q0 += tile_q) {
      n_items += num_qo_heads;
      kv_units += int64_t(num_qo_heads) * ((prefix + std::min(q0 + tile_q, ql) + kTileKV - 1) / kTileKV);
    }
  }
  // KV tiles per split (0: no split).
  const int64_t cus = num_cus > 0 ? num_cus : 256;
  const int64_t target = std::min<int64_t>(kSplitWaves * cus, kMaxSplitItems);
  int64_t chunk = 0;
  if (n_items > 0 && n_items < cus)
    chunk = std::max<int64_t>(kMinSplitTiles, (kv_units + target - 1) / target);
  const bool split_tiles = n_pairs < 2 * kXcds;
  std::vector<Group> groups;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t ql = q_indptr_host[b + 1] - q_indptr_host[b];
    if (ql == 0) continue;
    const int32_t prefix = kv_len_host[b] - ql;
    auto tile_cost = [&](int32_t q0) {
      return (int64_t(prefix) + std::min(q0 + tile_q, ql)) * ratio;
    };
    for (int32_t g = 0; g < num_kv_heads; ++g) {
      if (split_tiles) {
        for (int32_t q0 = 0; q0 < ql; q0 += tile_q)
          groups.push_back({b, g, q0, std::min(q0 + tile_q, ql), tile_cost(q0)});
      } else {
        int64_t cost = 0;
        for (int32_t q0 = 0; q0 < ql; q0 += tile_q) cost += tile_cost(q0);
        groups.push_back({b, g, 0, ql, cost});
      }
    }
  }
  std::stable_sort(groups.begin(), groups.end(),
                   [](const Group& x, const Group& y) { return x.cost > y.cost; });
  // Items of a group, split range by split range (the items of one range
  // read the same K/V), each range's tiles and heads together.
  std::vector<std::vector<int32_t>> lanes(kXcds);
  std::vector<int32_t> merges;
  int64_t load[kXcds] = {};
  int32_t slots = 0;
  for (const Group& g : groups) {
    const int x = int(std::min_element(load, load + kXcds) - load);
    load[x] += g.cost;
    const int32_t ql = q_indptr_host[g.seq + 1] - q_indptr_host[g.seq];
    const int32_t prefix = kv_len_host[g.seq] - ql;
    auto tile_end = [&](int32_t q0) { return prefix + std::min(q0 + tile_q, ql); };
    auto n_splits = [&](int32_t q0) {
      const int64_t units = (tile_end(q0) + kTileKV - 1) / kTileKV;
      return chunk > 0 ? int32_t((units + chunk - 1) / chunk) : 1;
    };
    int32_t max_splits = 1;
    for (int32_t q0 = g.t0; q0 < g.t1; q0 += tile_q) max_splits = std::max(max_splits, n_splits(q0));
    // First slot of each (tile, head) that is split.
    std::vector<int32_t> first_slot;
    for (int32_t q0 = g.t0; q0 < g.t1; q0 += tile_q) {
      const int32_t n = n_splits(q0);
      for (int32_t hq = g.hkv * ratio; hq < (g.hkv + 1) * ratio; ++hq) {
        first_slot.push_back(n > 1 ? slots : -1);
        if (n > 1) {
          merges.insert(merges.end(), {g.seq, q0, hq, slots, n});
          slots += n;
        }
      }
    }
    for (int32_t j = 0; j < max_splits; ++j) {
      size_t k = 0;
      for (int32_t q0 = g.t0; q0 < g.t1; q0 += tile_q) {
        const int32_t n = n_splits(q0);
        for (int32_t hq = g.hkv * ratio; hq < (g.hkv + 1) * ratio; ++hq, ++k) {
          if (j >= n) continue;
          const int32_t lo = n > 1 ? int32_t(j * chunk * kTileKV) : 0;
          const int32_t hi = (n > 1 && j + 1 < n) ? int32_t((j + 1) * chunk * kTileKV) : tile_end(q0);
          lanes[x].insert(lanes[x].end(), {g.seq, q0, hq, lo, hi, n > 1 ? first_slot[k] + j : -1});
        }
      }
    }
  }
  // Each XCD's workgroups in decreasing estimated duration (longest
  // processing time first: the XCD's CUs take them in this order as they
  // free up), interior KV tiles counting 1, diagonal tiles 1.6 and a
  // workgroup's start 3.5 (the kernel's measured per-tile and start-up
  // times). Ordering groups by their total left a step's single-tile items
  // (last chunks) behind cheaper tiles of longer groups, and the steps with
  // 1-3 workgroups per CU ended on them (chunked-prefill workload: +1-3%).
  for (auto& l : lanes) {
    const size_t n = l.size() / kRec;
    std::vector<std::pair<double, size_t>> order(n);
    for (size_t i = 0; i < n; ++i) {
      const int32_t* r = l.data() + kRec * i;
      const int32_t ql = q_indptr_host[r[0] + 1] - q_indptr_host[r[0]];
      const int32_t prefix = kv_len_host[r[0]] - ql;
      const int32_t t_lo = r[3] / kTileKV, t_hi = (r[4] + kTileKV - 1) / kTileKV;
      const int32_t t_int = std::max(t_lo, std::min(t_hi, (prefix + r[1] + 1) / kTileKV));
      order[i] = {3.5 + (t_int - t_lo) + 1.6 * (t_hi - t_int), i};
    }
    std::stable_sort(order.begin(), order.end(),
                     [](const std::pair<double, size_t>& a, const std::pair<double, size_t>& b) {
                       return a.first > b.first;
                     });
    std::vector<int32_t> sorted(l.size());
    for (size_t i = 0; i < n; ++i)
      std::copy(l.begin() + kRec * order[i].second, l.begin() + kRec * (order[i].second + 1),
                sorted.begin() + kRec * i);
    l.swap(sorted);
  }
  size_t depth = 0;
  for (const auto& l : lanes) depth = std::max(depth, l.size() / kRec);
  const int64_t need = int64_t(kRec) * int64_t(depth) * kXcds + int64_t(merges.size());
  if (need > plan_capacity) {
    set_error("prefill plan needs %lld ints, capacity %lld", (long long)need,
              (long long)plan_capacity);
    return KUNSERVE_ENOSPC;
  }
  // Workgroup L runs on XCD L % 8: item i of XCD x goes to L = 8 i + x.
  for (size_t i = 0; i < depth; ++i)
    for (int x = 0; x < kXcds; ++x) {
      int32_t* dst = plan_host + kRec * (i * kXcds + x);
      if (kRec * i < lanes[x].size()) {
        std::copy(lanes[x].begin() + kRec * i, lanes[x].begin() + kRec * (i + 1), dst);
      } else {
        std::fill(dst, dst + kRec, 0);
        dst[0] = -1;
        dst[5] = -1;
      }
    }
  std::copy(merges.begin(), merges.end(), plan_host + int64_t(kRec) * depth * kXcds);
  info->num_tiles = int32_t(depth * kXcds);
  info->tile_q = tile_q;
  info->head_dim = head_dim;
  info->plan_ints = int32_t(need);
  info->num_qo_heads = num_qo_heads;
  int32_t max_kv = 0;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t ql = q_indptr_host[b + 1] - q_indptr_host[b];
    if (ql > 0) max_kv = std::max(max_kv, kv_len_host[b]);
  }
  info->max_kv_len = max_kv;
  info->num_merge = int32_t(merges.size() / kMergeRec);
  info->num_slots = slots;
  info->kv_chunk = int32_t(chunk * kTileKV);
  return KUNSERVE_OK;
}

extern "C" int64_t kunserve_prefill_workspace_bytes(const kunserve_prefill_plan_info* info) {
  if (!info) return -1;
  return int64_t(info->num_slots) * info->tile_q * (info->head_dim + 2) * int64_t(sizeof(float));
}

extern "C" int kunserve_paged_prefill(const kunserve_kv_pool* pool, int32_t layer,
                                      const kunserve_page_table* table,
                                      const int32_t* q_indptr_dev, const int32_t* q_start_dev,
                                      const kunserve_tensor3* q,
                                      kunserve_tensor3* out, int32_t num_qo_heads,
                                      float sm_scale, const int32_t* plan_dev,
                                      const kunserve_prefill_plan_info* info,
                                      void* workspace_dev, int64_t workspace_bytes,
                                      kunserve_stream_t stream) {
  clear_error();
  int rc = check_pool(pool, true);
  if (rc) return rc;
  KSV_CHECK_ARG(table && q && out && info, "null argument");
  KSV_CHECK_ARG(layer >= 0 && layer < pool->num_layers, "layer %d outside [0, %d)", layer,
                pool->num_layers);
  KSV_CHECK_ARG(std::isfinite(sm_scale) && sm_scale > 0.f,
                "sm_scale %g must be finite and positive", double(sm_scale));
  if (!prefill_head_dim_ok(pool->head_dim)) {
    set_error("prefill supports head_dim 64, 128 and 256, got %d", pool->head_dim);
    return KUNSERVE_EUNSUPPORTED;
  }
  KSV_CHECK_ARG(num_qo_heads > 0 && num_qo_heads % pool->num_kv_heads == 0,
                "num_qo_heads %d not a multiple of num_kv_heads %d", num_qo_heads,
                pool->num_kv_heads);
  KSV_CHECK_ARG(info->head_dim == pool->head_dim && info->tile_q == tile_q_for(pool->head_dim),
                "plan made for head_dim %d (tile %d), pool has head_dim %d", info->head_dim,
                info->tile_q, pool->head_dim);
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
  const int64_t ws_need = kunserve_prefill_workspace_bytes(info);
  if (info->num_slots > 0 && (!workspace_dev || workspace_bytes < ws_need)) {
    set_error("prefill workspace holds %lld bytes, %lld needed", (long long)workspace_bytes,
              (long long)ws_need);
    return KUNSERVE_ENOSPC;
  }
  PrefillArgs a{};
  a.q = static_cast<const f16*>(q->data);
  a.q_tok = q->token_stride;
  a.q_head = q->head_stride;
  a.out = static_cast<f16*>(out->data);
  a.o_tok = out->token_stride;
  a.o_head = out->head_stride;
  a.k = static_cast<const f16*>(pool->k) + int64_t(layer) * pool->layer_stride;
  a.v = static_cast<const f16*>(pool->v) + int64_t(layer) * pool->layer_stride;
  // Gathers address a page with one 32 x 32 -> 64-bit multiply-add.
  if (pool->page_stride > int64_t(UINT32_MAX) ||
      int64_t(pool->page_size) * pool->token_stride > int64_t(UINT32_MAX)) {
    set_error("prefill needs page_stride (%lld) and page_size x token_stride below 2^32",
              (long long)pool->page_stride);
    return KUNSERVE_EUNSUPPORTED;
  }
  a.page_stride = uint32_t(pool->page_stride);
  a.head_stride = pool->head_stride;
  a.token_stride = uint32_t(pool->token_stride);
  a.num_pages = int32_t(pool->num_pages);
  a.page_shift = __builtin_ctz(pool->page_size);
  a.indptr = table->indptr_dev;
  a.indices = table->indices_dev;
  a.kv_len = table->kv_len_dev;
  a.q_indptr = q_indptr_dev;
  a.q_start = q_start_dev;
  a.tiles = plan_dev;
  a.part_o = static_cast<float*>(workspace_dev);
  a.part_ml = a.part_o ? a.part_o + int64_t(info->num_slots) * info->tile_q * pool->head_dim
                       : nullptr;
  a.ratio = num_qo_heads / pool->num_kv_heads;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  const int64_t pages_needed = (int64_t(info->max_kv_len) + pool->page_size - 1) / pool->page_size;
  MergeArgs m{};
  m.merges = plan_dev + int64_t(kRec) * info->num_tiles;
  m.part_o = a.part_o;
  m.part_ml = a.part_ml;
  m.q_indptr = q_indptr_dev;
  m.q_start = q_start_dev;
  m.out = a.out;
  m.o_tok = a.o_tok;
  m.o_head = a.o_head;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (pool->dtype == KUNSERVE_DTYPE_BF16)
    return run_prefill_dim<bf16>(pool->head_dim, a, m, info->num_tiles, info->num_merge,
                             pages_needed <= kMaxStagedPages, s);
  return run_prefill_dim<f16>(pool->head_dim, a, m, info->num_tiles, info->num_merge,
                              pages_needed <= kMaxStagedPages, s);
}

// ------------------------------------------------------------ calibration
// The rate this part sustains on the prefill kernels' MFMA: two waves per
// SIMD issue independent 32x32x16 MFMAs on per-lane operands held in
// registers. The operands' bits set the power the matrix cores draw, and so
// the clock the part holds under its power limit: random operands draw what
// attention operands draw, constant ones much less.
namespace kunserve {
namespace {

constexpr int kMfmaProbeThreads = 512;

template <typename T>
__global__ __launch_bounds__(kMfmaProbeThreads) void mfma_probe_kernel(const T* operands, float* sink,
                                                                       int iterations) {
  typedef typename Vec<T>::v8 V8;
  const int64_t t = int64_t(blockIdx.x) * kMfmaProbeThreads + threadIdx.x;
  const V8 x = *reinterpret_cast<const V8*>(operands + 16 * t);
  const V8 y = *reinterpret_cast<const V8*>(operands + 16 * t + 8);
  f32x16 a0 = {}, a1 = {};
  for (int i = 0; i < iterations; ++i) {
    a0 = mfma32(x, y, a0);
    a1 = mfma32(y, x, a1);
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += a0[e] + a1[e];
  sink[t] = s;
}

}  // namespace
}  // namespace kunserve

extern "C" int kunserve_mfma_probe(int32_t dtype, const void* operands_dev, float* sink_dev,
                                   int32_t num_workgroups, int32_t iterations,
                                   kunserve_stream_t stream) {
  using namespace kunserve;
  clear_error();
  KSV_CHECK_ARG(dtype == KUNSERVE_DTYPE_F16 || dtype == KUNSERVE_DTYPE_BF16,
                "dtype %d is not KUNSERVE_DTYPE_F16 or KUNSERVE_DTYPE_BF16", dtype);
  KSV_CHECK_ARG(num_workgroups > 0 && iterations > 0,
                "num_workgroups (%d) and iterations (%d) must be positive", num_workgroups,
                iterations);
  KSV_CHECK_ARG(operands_dev && sink_dev && aligned16(operands_dev) && aligned16(sink_dev),
                "null or misaligned buffer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == KUNSERVE_DTYPE_BF16)
    mfma_probe_kernel<bf16><<<num_workgroups, kMfmaProbeThreads, 0, s>>>(
        static_cast<const bf16*>(operands_dev), sink_dev, iterations);
  else
    mfma_probe_kernel<f16><<<num_workgroups, kMfmaProbeThreads, 0, s>>>(
        static_cast<const f16*>(operands_dev), sink_dev, iterations);
  KSV_CHECK_LAUNCH();
  return KUNSERVE_OK;
}
