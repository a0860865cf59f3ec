// Verify attention for gfx950: MQA of the k+1 (or tree) query positions of a
// speculative-decoding step against each batch row's key/value table.
//
// Semantics follow the reference's PyTorch form (pytorch_kernels.py:98-121
// exact attention; :149-153,171-187 window and sink; attention.py:74-82 the
// masked dense form): FP32 scores q.k*scale, FP32 softmax, output in the
// input dtype.
//
// MFMA kernel (bf16, head width 64 or 128).  The H query heads of the T
// positions of one batch row are stacked as R = T*H rows (row r = t*H + h),
// so the single shared K/V head is read once per query group and feeds
// 16-row MFMA blocks.  Each workgroup (4 wavefronts) owns one part ("split")
// of a batch row's visible key range; each wavefront streams its own 16-row
// key/value blocks straight from HBM with 16-byte loads, one block ahead:
//
//   S^T[kv, q] = K[kv, :] . Q[q, :]     v_mfma_f32_16x16x32_bf16, K as the A
//                                      operand (one key row per lane), Q^T
//                                      held in registers as the B operand
//   online softmax per query row        each lane holds 4 keys x 1 query row;
//                                      max/sum across the 4 lane groups
//   O^T[c, q] += V^T[c, kv] . P^T[kv,q] v_mfma_f32_16x16x16_bf16: the S^T
//                                      accumulator is already P^T's operand
//                                      layout; V^T comes from a per-wavefront
//                                      LDS staging buffer read transposed
//
// The four wavefronts of a workgroup are merged through LDS at the end; the
// splits of one batch row are merged by a second kernel (log-sum-exp
// combine, fixed order, so results do not depend on scheduling).
//
// Generic kernel (fp32 or bf16, any head width <= 256, chosen rows): one
// wavefront per (batch row, query position, head), one key row per lane,
// the reference algorithm in FP32 with an online softmax.  It is the fp32
// path and the chosen-row (sparse) path.
#include "wptv_common.h"

#include <climits>
#include <mutex>
#include <type_traits>

namespace wptv {
namespace {

constexpr float kNegInf = -__builtin_inff();

struct Bounds {
  int lo, hi;  // inclusive key-row range a query sees (hi < lo: none)
};

// The key rows query position t of batch row b sees, before the tree mask.
// A batch row's query positions: p[t], or (a draft tree given without
// positions) node t at base + t.
// p[i] of an input that no kernel of the launch writes, read as constant
// memory: a scalar load where i is uniform (on the scalar counter, apart from
// the vector-memory counter the kernels' DMA runs on, which the compiler's own
// waits cannot count), a vector load where it is not.
template <typename T>
__device__ __forceinline__ T const_load(const T* p, int64_t i) {
  return ((const __attribute__((address_space(4))) T*)(uintptr_t)p)[i];
}

struct QueryPos {
  const int64_t* p;
  int64_t base;
  __device__ __forceinline__ int64_t at(int t) const { return p ? const_load(p, t) : base + t; }
};

__device__ __forceinline__ QueryPos query_pos(const int64_t* positions, const int64_t* tree_base, int b, int T) {
  return positions ? QueryPos{positions + (int64_t)b * T, 0} : QueryPos{nullptr, tree_base[b]};
}

__device__ __forceinline__ Bounds query_bounds(const QueryPos& pos_b, int t, int window, int N) {
  const int64_t p = pos_b.at(t);
  int64_t hi = p < (int64_t)N - 1 ? p : (int64_t)N - 1;
  int64_t lo = window > 0 ? p - window + 1 : 0;
  if (lo < 0) lo = 0;
  Bounds r;
  r.lo = (int)lo;
  r.hi = hi < lo ? (int)lo - 1 : (int)hi;
  return r;
}

// The union [u_lo, u_hi] of the key rows that positions t_first .. t_last
// see (u_hi < u_lo: none), uniform.  A lane per position, so the positions
// come in by one vector load instead of one dependent scalar load each; every
// lane of the wavefront must be active.
__device__ __forceinline__ void union_bounds(const QueryPos& pos_b, int t_first, int t_last, int window, int N,
                                             int lane, int& u_lo, int& u_hi) {
  int lo_l = INT_MAX, hi_l = -1;
  for (int t0 = t_first; t0 <= t_last; t0 += 64) {
    if (t0 + lane <= t_last) {
      const Bounds bt = query_bounds(pos_b, t0 + lane, window, N);
      if (bt.hi >= bt.lo) {
        lo_l = min(lo_l, bt.lo);
        hi_l = max(hi_l, bt.hi);
      }
    }
  }
  u_lo = __builtin_amdgcn_readfirstlane(wave_min_i32(lo_l));
  u_hi = __builtin_amdgcn_readfirstlane(wave_max_i32(hi_l));
}

__device__ __forceinline__ bool tree_visible(int n, int64_t tbase, uint64_t anc) {
  if ((int64_t)n < tbase) return true;
  const int64_t node = (int64_t)n - tbase;
  return node < 64 && ((anc >> node) & 1ull);
}

// Where logical row n (a token's position) of batch row b sits in the table:
// physical row (n - base[b]) & mask.  The default (base NULL, mask all ones)
// is token p at row p; a window layer's ring of 2^r rows per batch row has
// mask 2^r - 1; a table that starts at a later token has base[b] = that
// token's position.
struct RowMap {
  const int64_t* base;
  uint32_t mask;
};

// The table row of batch row b's first ring slot (a scalar load).
__device__ __forceinline__ int row_base(const RowMap& m, int b) { return m.base ? (int)const_load(m.base, b) : 0; }

// A window or sparse layer's output gate (attention.py:128-130): the output
// o (rounded to bf16, the attention's dtype) times sigmoid(gate) (rounded to
// bf16, as torch.sigmoid of a bf16 tensor), rounded again.  Row (b*T + t) of
// the gate at g + (b*T + t)*stride, head h's columns at + h*c; g NULL: none.
struct OutGate {
  const void* g;  // in the attention's dtype
  int64_t stride;
  template <typename E>
  __device__ __forceinline__ const E* row(int b, int T, int r, int H, int C) const {
    return g ? static_cast<const E*>(g) + ((int64_t)b * T + r / H) * stride + (int64_t)(r % H) * C : nullptr;
  }
};

__device__ __forceinline__ float gate_factor(unsigned short g) {
  return bf16_to_f32(f32_to_bf16(1.f / (1.f + __expf(-bf16_to_f32(g)))));
}

// o rounded to bf16, times the gate factor, rounded again.
__device__ __forceinline__ unsigned short gated_bf16(float o, unsigned short g) {
  return f32_to_bf16(bf16_to_f32(f32_to_bf16(o)) * gate_factor(g));
}

// Merges the parts of one query row's 8 columns c8 .. c8 + 7: fixed split
// order, log-sum-exp weights, the sink (log2 units; -inf: none) joining the
// denominator.  Part s of the row is at row0 + s * stride (bf16 output,
// normalized within the part, and its log2-sum-exp).  The parts are read
// eight at a time, every load of a group issued before any is used, with a
// running maximum across groups.  Writes the 8 outputs and, when lse is
// given and c8 == 0, the row's natural-log log-sum-exp.  grow: the row's
// output gate (NULL: none).  dst8: where the 8 outputs go.
__device__ __forceinline__ void merge_parts(const unsigned short* __restrict__ part_o,
                                            const float* __restrict__ part_lse, int64_t row0, int64_t stride,
                                            int splits, int C, int c8, float sink_log2,
                                            unsigned short* __restrict__ dst8, float* __restrict__ lse,
                                            const unsigned short* __restrict__ grow) {
  constexpr int kGroup = 8;
  float M = kNegInf, L = 0.f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < splits; s0 += kGroup) {
    float ls[kGroup];
    u16x8 po[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int64_t prow = row0 + (int64_t)(s0 + u) * stride;
      const bool in = s0 + u < splits;
      ls[u] = in ? part_lse[prow] : kNegInf;
      po[u] = in ? *reinterpret_cast<const u16x8*>(part_o + prow * C + c8) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    float m = M;
#pragma unroll
    for (int u = 0; u < kGroup; ++u) m = fmaxf(m, ls[u]);
    if (m == kNegInf) continue;  // nothing seen yet
    const float f = M == kNegInf ? 0.f : exp2f(M - m);
    L *= f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= f;
    M = m;
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      if (ls[u] == kNegInf) continue;
      const float wgt = exp2f(ls[u] - M);
      L += wgt;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += wgt * bf16_to_f32(po[u][e]);
    }
  }
  if (sink_log2 != kNegInf) {
    const float M2 = fmaxf(M, sink_log2);
    const float f = M == kNegInf ? 0.f : exp2f(M - M2);
    L = L * f + exp2f(sink_log2 - M2);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= f;
    M = M2;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  u16x8 res;
  if (grow) {
    const u16x8 gv = *reinterpret_cast<const u16x8*>(grow + c8);
#pragma unroll
    for (int e = 0; e < 8; ++e) res[e] = gated_bf16(acc[e] * inv, gv[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) res[e] = f32_to_bf16(acc[e] * inv);
  }
  *reinterpret_cast<u16x8*>(dst8) = res;
  if (lse && c8 == 0) *lse = L > 0.f ? (M + log2f(L)) * kLn2 : kNegInf;
}

// The key rows [u_lo, u_hi] in `splits` parts of whole 32-row tiles, as even
// as they go (the first full % splits parts one tile more); the rows past the
// last whole tile join the last part as a partial tile, whose DMA re-reads
// its last row for the rest.  An empty part has s_hi < s_lo.
__device__ __forceinline__ void split_range(int u_lo, int u_hi, int splits, int split, int& s_lo, int& s_hi) {
  const int U = u_hi - u_lo + 1;
  const int full = U / 32, rem = U % 32;
  const int q = full / splits, r = full % splits;
  const int first = split * q + min(split, r);
  const int tiles = q + (split < r ? 1 : 0);
  s_lo = u_lo + 32 * first;
  s_hi = s_lo + 32 * tiles - 1 + (split == splits - 1 ? rem : 0);
}

// ---------------------------------------------------------------------------
// MFMA kernel
// ---------------------------------------------------------------------------

template <int C>
struct Tile {
  static constexpr int kSteps = C / 32;             // k-steps of the QK^T product (16x16x32)
  static constexpr int kCBlocks = C / 16;           // 16-wide column blocks of O
  static constexpr int kHalf = 16 * C;              // one 16-row block of K or V (bf16 elements)
  static constexpr int kElems = 4 * kHalf;          // a 32-row tile: K rows 0-15, 16-31, then V rows 0-15, 16-31
  static constexpr int kLoads = kElems * 2 / 1024;  // 1 KiB DMA instructions per tile (16 at head width 128)
  static constexpr int kPerHalf = C / 32;           // DMA instructions per 16-row half
  static constexpr int kSlots = 4;                  // tiles in each key-set's ring
};
constexpr int kKeySets = 2;  // wavefront sets that take alternate tiles of the workgroup's key range

// The swizzle of the row-block kernel's row-major tile halves (chunk x of row
// r at unit (C / 8) r + (x ^ tile_sigma(r))): the 16 rows of a K operand read
// land on 16 distinct bank groups, and so do the chunk pairs 2cb, 2cb + 1 of
// rows 0-7 (8-15) that a transposed V read takes.
template <int C>
__device__ __forceinline__ int tile_sigma(int r) {
  if constexpr (C == 128) return 2 * (r & 7) + (r >> 3);
  else return 2 * ((r >> 1) & 3) + (r >> 3);
}

// The 32-row kernel's swizzle of its V halves (head width 128): its
// transposed reads take, in each half of the wavefront, rows 4 i .. 4 i + 3
// at chunks 4 cb + a (a < 4), and 4 (r % 4) moves those 16 (row, chunk)
// pairs onto 16 distinct bank groups.
__device__ __forceinline__ int v_sigma(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// A row's softmax reference maximum is its first finite tile maximum and
// moves only when a later tile's maximum exceeds it by more than this many
// powers of two (p then stays below 2^32, far inside the fp32 and bf16
// range; the stale maximum stays the reference for p and l, so the result is
// exact either way).  Moving it from -inf needs no rescale (O and l are still
// 0); a real rescale is rare and done in one uniform branch.
constexpr float kRescaleLog2 = 32.f;

__device__ __forceinline__ bf16x8 pack_bf16x8(const float (&p)[8]) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = static_cast<__bf16>(p[e]);
  return r;
}

// The larger of two scores: IEEE maximum (NaN propagates), one v_maximum3_f32
// for up to three operands with no canonicalisation of its inputs (fmaxf
// would first quiet each input with an extra v_max).
__device__ __forceinline__ float score_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max / sum over the four 16-lane groups (lanes j, j+16, j+32, j+48).
__device__ __forceinline__ float group_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = score_max(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return score_max(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float group_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One workgroup per (batch row, row group, key split): kKeySets x MB
// wavefronts; wavefront (s, mb) holds m-block mb (16 query rows) and takes the
// 32-row key tiles s, s + 2, ... of the split.  The tiles of a key set are
// DMA'd into its LDS ring by its first DMAW wavefronts and read by all MB of
// them; a workgroup barrier per iteration hands them over.  The parameters
// the first key range depends on come first: gfx950 preloads a kernel's first
// 14 argument dwords into SGPRs, so the positions load is issued at once and
// the rest of the arguments arrive meanwhile.
template <int C, int MB, bool TREE>
__global__ __launch_bounds__(kKeySets * MB * 64, 1) void verify_attention_mfma(
    const int64_t* __restrict__ positions, const int64_t* __restrict__ tree_base, int xcd_map, int groups,
    int splits, int T, int H, int N, int window, int range_from_positions, const unsigned short* __restrict__ k,
    int64_t ksb, int64_t ksn, const unsigned short* __restrict__ v, int64_t vsb, int64_t vsn,
    const unsigned short* __restrict__ q, const uint64_t* __restrict__ ancestors, const float* __restrict__ sink,
    float scale_log2, RowMap rows, OutGate gate, unsigned short* __restrict__ out, int out_fm,
    float* __restrict__ lse_out, unsigned short* __restrict__ part_o, float* __restrict__ part_lse) {
  using G = Tile<C>;
  constexpr int kRows = 16 * MB;
  constexpr int kXC = C / 8;  // 16-byte chunks per key or value row
  constexpr int DMAW = MB >= 4 ? 4 : (MB >= 2 ? 2 : 1);  // wavefronts of a key set that issue its DMA
  constexpr int kCnt = G::kLoads / DMAW;                 // DMA instructions per such wavefront and tile
  constexpr int kRing = G::kSlots * G::kElems;           // elements of one key set's ring
  constexpr int kPitch = C + 4;                          // merge buffer row pitch (floats): distinct banks
  static_assert(G::kLoads % DMAW == 0, "DMA split");
  static_assert(MB * (16 * kPitch + 32) * 4 <= kKeySets * kRing * 2, "the merge buffer reuses the rings");
  __shared__ __attribute__((aligned(16))) unsigned short lds[kKeySets * kRing];
  __shared__ __attribute__((aligned(16))) unsigned short qlds[MB * 16 * C];  // each m-block's queries

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kset = wid / MB, mb = wid % MB;
  const int j = lane & 15;  // this lane's column: query row (S^T, O^T) or key row (K operand)
  const int g = lane >> 4;  // lane group 0..3

  // Workgroups are dealt to the 8 XCDs in turn: every group and split of a
  // batch row share one XCD (its L2), where several groups read the same
  // keys and values
  int unit, split;
  {
    const int L = blockIdx.x;
    if (xcd_map) {
      const int slot = L >> 3, per_row = groups * splits;
      const int bb = (L & 7) + 8 * (slot / per_row), rem = slot % per_row;
      unit = bb * groups + rem / splits;
      split = rem % splits;
    } else {
      unit = L / splits;
      split = L % splits;
    }
  }
  const int b = unit / groups;
  const int grp = unit % groups;
  const int R = T * H;
  const int r_base = grp * kRows;
  const QueryPos pos_b = query_pos(positions, tree_base, b, T);

  // The key rows this workgroup's queries can see: the positions come in by
  // one vector load (a lane each), waited for here, before any DMA (the
  // compiler's waits on vector memory cannot count the DMA, so a vector load
  // waited for among the DMA would drain the DMA with it).
  const int r = r_base + 16 * mb + j;
  const bool real = r < R;
  int u_lo = 0, u_hi = N - 1;
  if (range_from_positions)
    union_bounds(pos_b, r_base / H, (min(r_base + kRows, R) - 1) / H, window, N, lane, u_lo, u_hi);
  int s_lo = 0, s_hi = -1;
  if (u_hi >= u_lo) split_range(u_lo, u_hi, splits, split, s_lo, s_hi);
  const int ntiles = s_hi >= s_lo ? (s_hi - s_lo + 1 + 31) / 32 : 0;
  const int niter = (ntiles + kKeySets - 1) / kKeySets;       // workgroup iterations
  const int mine = ntiles > kset ? (ntiles - kset + kKeySets - 1) / kKeySets : 0;  // tiles of this key set

  // DMA: instruction ii of a tile covers whole rows of one half, 64 / XC
  // rows of XC = C / 8 16-byte chunks (part = ii / kPerHalf: K rows 0-15,
  // K rows 16-31, V rows 0-15, V rows 16-31), so each instruction reads
  // 1 KiB of consecutive rows (measured on the stream alone: 12.4 us for the
  // 64 MB of batch 32 x 4096 against 14.0 us reading 16 rows x 64 bytes).
  // LDS layout of a half, row-major with a swizzle: chunk x of row r at
  // unit XC r + (x ^ tile_sigma(r)); lane l of the instruction fills unit
  // 64 (ii % kPerHalf) + l, so it fetches the chunk whose swizzled place
  // that is.
  const i32x4 krs = buffer_resource(k + (int64_t)b * ksb);
  const i32x4 vrs = buffer_resource(v + (int64_t)b * vsb);
  const uint32_t krow_bytes = (uint32_t)ksn * 2u, vrow_bytes = (uint32_t)vsn * 2u;
  unsigned short* const ring = lds + kset * kRing;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  const bool dma_wave = mb < DMAW;
  const int rbase = row_base(rows, b);
  auto issue = [&](int it) {  // this wavefront's share of the key set's tile of iteration it
    const int tile = kset + it * kKeySets;
    const uint32_t slot = ring_lds + (uint32_t)(it % G::kSlots) * (G::kElems * 2);
#pragma unroll
    for (int c = 0; c < kCnt; ++c) {
      const int ii = mb * kCnt + c;
      const int part = ii / G::kPerHalf, quarter = ii % G::kPerHalf;
      const int row = quarter * (64 / kXC) + lane / kXC;  // the row of the half this lane fills
      const int x = (lane % kXC) ^ tile_sigma<C>(row);    // the chunk that belongs there
      int n = s_lo + tile * 32 + 16 * (part & 1) + row;
      n = n < s_hi ? n : s_hi;  // rows past the split are masked; read a valid one
      const uint32_t phys = (uint32_t)(n - rbase) & rows.mask;
      const uint32_t off = phys * (part < 2 ? krow_bytes : vrow_bytes) + 16u * x;
      const uint32_t dst = __builtin_amdgcn_readfirstlane(slot + part * (G::kHalf * 2) + 1024u * quarter);
      i32x4 rs;
#pragma unroll
      for (int e = 0; e < 4; ++e) rs[e] = __builtin_amdgcn_readfirstlane(part < 2 ? krs[e] : vrs[e]);
      // a full-context table read by this query group only: non-temporal (several groups, or the
      // next step's reading of a sliding window, reuse them through the caches)
      if (groups == 1 && window == 0)
        dma_16B_nt(rs, off, dst);
      else
        dma_16B(rs, off, dst);
    }
  };
  // The queries go out first (DMA into qlds, each m-block laid out like a
  // key half, so that the Q^T operand of k-step s is unit 64s + lane; the
  // first key set loads them, the second reads them after the first
  // barrier), then the first tiles.  Waiting for tile 0 then implies the
  // queries.  Every other load of the kernel was waited for before this
  // point, so the compiler needs no vector-memory wait of its own from here
  // on (it cannot count the DMA).
  if (kset == 0) {
    i32x4 qrs = buffer_resource(q + (int64_t)b * R * C);
#pragma unroll
    for (int e = 0; e < 4; ++e) qrs[e] = __builtin_amdgcn_readfirstlane(qrs[e]);
    const uint32_t qoff = (uint32_t)(real ? r : R - 1) * (uint32_t)(C * 2) + 16u * g;  // a padding row reads row R-1
    const uint32_t qdst = __builtin_amdgcn_readfirstlane(lds_address(qlds + mb * 16 * C));
#pragma unroll
    for (int s = 0; s < G::kSteps; ++s) dma_16B(qrs, qoff + 64u * s, qdst + 1024u * s);
  }
  if (dma_wave) {
#pragma unroll
    for (int it = 0; it < G::kSlots - 1; ++it)
      if (it < mine) issue(it);
  }
  // Per-row bounds: the wavefront's 16 rows span positions t_first..t_last;
  // each position is read with a uniform (scalar) load, on the scalar counter,
  // and the lanes of that position take it.  f_lo, f_hi: the rows every query
  // of the wavefront sees.
  int lo = 0, hi = -1;
  uint64_t anc = 0;
  int f_lo = 0, f_hi = INT_MAX;
  const int64_t tbase = TREE ? tree_base[b] : (int64_t)INT_MAX;
  {
    const int w_first = r_base + 16 * mb;
    if (w_first < R) {
      const int t_first = w_first / H, t_last = (min(w_first + 16, R) - 1) / H;
      const int my_t = real ? r / H : -1;
      for (int t = t_first; t <= t_last; ++t) {
        const Bounds bt = query_bounds(pos_b, t, window, N);
        f_lo = max(f_lo, bt.lo);
        f_hi = min(f_hi, bt.hi);
        if (my_t == t) {
          lo = bt.lo;
          hi = min(bt.hi, s_hi);
        }
        if constexpr (TREE) {
          const uint64_t a = const_load(ancestors, t);
          if (my_t == t) anc = a;
        }
      }
    } else {
      f_hi = -1;
    }
    if (TREE && tbase <= (int64_t)f_hi) f_hi = (int)tbase - 1;
    f_hi = min(f_hi, s_hi);
  }

  bf16x8 qf[G::kSteps];
  f32x4 o[G::kCBlocks];
#pragma unroll
  for (int cb = 0; cb < G::kCBlocks; ++cb) o[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;
  // the transposed V reads: lane 16g + 4rr + qq addresses row 4g + rr,
  // columns 4qq..4qq+3 of the 16-column block cb, i.e. chunk 2cb + (qq >> 1)
  // (= 2cb ^ (qq >> 1)), element 4 (qq & 1) of it
  const int tr_row = 4 * g + ((lane >> 2) & 3);
  const int tr_base = 8 * kXC * tr_row + 4 * (lane & 1);
  const int tr_y = ((lane & 3) >> 1) ^ tile_sigma<C>(tr_row);
  // the K operand of k-step s: row j, chunk 4s + g (= 4s ^ g)
  const int k_base = 8 * kXC * j;
  const int k_y = g ^ tile_sigma<C>(j);

  // Waits for this key set's tile of iteration t (each DMA wavefront for its
  // own loads, at most `later` tiles' loads still in flight behind it), then
  // a bare workgroup barrier: a fence here would wait for the later tiles too.
  auto arrive = [&](int t, int later) {
    if (dma_wave && t < mine) {
      if (later >= 2)
        wait_vmcnt<2 * kCnt>();
      else if (later == 1)
        wait_vmcnt<kCnt>();
      else
        wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // S^T = K . Q^T of a tile's two 16-row halves: lane (j, g) reads key row j, chunk 4s + g.
  auto qk = [&](int t, f32x4& s0, f32x4& s1) {
    const unsigned short* st = ring + (t % G::kSlots) * G::kElems;
    s0 = f32x4{0.f, 0.f, 0.f, 0.f};
    s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < G::kSteps; ++s) {
      const int k_off = k_base + 8 * ((4 * s) ^ k_y);
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(st + k_off);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(st + G::kHalf + k_off);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[s], s1, 0, 0, 0);
    }
  };
  // The probabilities of a tile against the running maximum, and O^T += V^T . P^T.
  auto accumulate = [&](int t, const f32x4& s0, const f32x4& s1) {
    const unsigned short* st = ring + (t % G::kSlots) * G::kElems;
    const int n0 = s_lo + (kset + t * kKeySets) * 32;
    float x[8];  // raw scores (the scale is positive: maxima commute with it)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = s0[i];
      x[4 + i] = s1[i];
    }
    if (!(n0 >= f_lo && n0 + 31 <= f_hi)) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = n0 + 16 * h + 4 * g + i;
          bool vis = n >= lo && n <= hi;
          if constexpr (TREE) vis = vis && tree_visible(n, tbase, anc);
          x[4 * h + i] = vis ? x[4 * h + i] : kNegInf;
        }
    }
    const float bm = group_max(score_max(score_max(score_max(x[0], x[1]), score_max(x[2], x[3])),
                                         score_max(score_max(x[4], x[5]), score_max(x[6], x[7])))) *
                     scale_log2;
    const bool grow = bm > m_run + kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow && m_run != kNegInf)) {
      const float alpha = (grow && m_run != kNegInf) ? __builtin_amdgcn_exp2f(m_run - bm) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < G::kCBlocks; ++cb) o[cb] *= alpha;
    }
    m_run = grow ? bm : m_run;
    // a row with no visible key so far has every score at -inf: any finite
    // reference gives p = 0
    const float neg_m = m_run == kNegInf ? 0.f : -m_run;
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(fmaf(x[e], scale_log2, neg_m));
    l_run += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    // P^T operand: lane (j, g) holds k-index 8g + e = key 4g + e of the first
    // half (e < 4), key 16 + 4g + e - 4 of the second; the V^T operand holds
    // the same keys at column cb*16 + j, two transposed 4-row reads.
    const bf16x8 pt = pack_bf16x8(p);
    const unsigned short* vs = st + 2 * G::kHalf + tr_base;
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const int cofs = 8 * ((2 * cb) ^ tr_y);
      const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vs + cofs));
      const s16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vs + G::kHalf + cofs));
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      const s16x8 vt = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
      o[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vt), pt, o[cb], 0, 0, 0);
    }
  };

  // Software pipeline: iteration it multiplies the next tile's keys (QK^T on
  // the matrix cores) before the softmax and PV of its own tile, whose VALU
  // work then overlaps them.  Tiles it (PV) and it + 1 (QK) occupy two slots,
  // it + 2 and it + 3 are in flight.
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
  // a first-set wavefront that waits for no tile waits for its queries here
  if (kset == 0 && !(dma_wave && mine > 0)) wait_vmcnt<0>();
  arrive(0, min(G::kSlots - 2, mine - 1));  // tile 0 and every m-block's queries are in LDS
#pragma unroll
  for (int s = 0; s < G::kSteps; ++s)
    qf[s] = *reinterpret_cast<const bf16x8*>(qlds + mb * 16 * C + 512 * s + 8 * lane);
  if (mine > 0) qk(0, s0, s1);
  // Iteration it: the scores of tile it + 1 into (n0, n1), the softmax and PV
  // of tile it from (c0, c1).  Two iterations per trip, the score registers
  // taking turns, so that no copy moves them.
  auto iteration = [&](int it, const f32x4& c0, const f32x4& c1, f32x4& n0, f32x4& n1) {
    arrive(it + 1, min(1, mine - 2 - it));  // every wavefront is done with iteration it - 1
    if (dma_wave && it + G::kSlots - 1 < mine) issue(it + G::kSlots - 1);
    if (it + 1 < mine) qk(it + 1, n0, n1);
    if (it < mine) accumulate(it, c0, c1);
  };
  f32x4 n0 = {0.f, 0.f, 0.f, 0.f}, n1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int it = 0; it < niter; it += 2) {
    iteration(it, s0, s1, n0, n1);
    if (it + 1 < niter) iteration(it + 1, n0, n1, s0, s1);
  }
  wait_vmcnt<0>();
  l_run = group_sum(l_run);

  // ---- merge the key sets (the merge buffer reuses the rings) ----
  __syncthreads();
  float* mbuf = reinterpret_cast<float*>(lds) + mb * (16 * kPitch + 32);  // this m-block's O, then m, l
  if (kset == 1) {
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb)
      *reinterpret_cast<f32x4*>(mbuf + j * kPitch + cb * 16 + 4 * g) = o[cb];
    if (g == 0) {
      mbuf[16 * kPitch + j] = m_run;
      mbuf[16 * kPitch + 16 + j] = l_run;
    }
  }
  __syncthreads();
  if (kset != 0) return;
  {
    const float m1 = mbuf[16 * kPitch + j], l1 = mbuf[16 * kPitch + 16 + j];
    const float M = fmaxf(m_run, m1);
    const float a0 = m_run == kNegInf ? 0.f : exp2f(m_run - M);
    const float a1 = m1 == kNegInf ? 0.f : exp2f(m1 - M);
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb)
      o[cb] = o[cb] * a0 + *reinterpret_cast<const f32x4*>(mbuf + j * kPitch + cb * 16 + 4 * g) * a1;
    l_run = l_run * a0 + l1 * a1;
    m_run = M;
  }
  if (!real) return;

  // Final statistics of the row (the sink joins the denominator when the
  // split is the whole range), then the output or this split's part.
  float M = m_run, L = l_run, f = 1.f;
  if (splits == 1 && sink) {
    const float sl = sink[r % H] * kLog2e;
    const float M2 = fmaxf(M, sl);
    f = (M == kNegInf) ? 0.f : exp2f(M - M2);
    L = L * f + exp2f(sl - M2);
    M = M2;
  }
  const float scale_out = L > 0.f ? f / L : 0.f;
  const float lse2 = L > 0.f ? M + log2f(L) : kNegInf;
  if (splits == 1) {
    typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
    unsigned short* orow = out + ((int64_t)b * R + r) * C;
    const unsigned short* grow = gate.row<unsigned short>(b, T, r, H, C);
    // out_fm > 0: the output [B T, H C] in the fm layout with out_fm row blocks
    const int fm_row = b * T + r / H, fm_col = (r % H) * C;
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const f32x4 val = o[cb] * scale_out;
      u16x4 res;
      if (grow) {
        const u16x4 gv = *reinterpret_cast<const u16x4*>(grow + cb * 16 + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) res[e] = gated_bf16(val[e], gv[e]);
      } else {
        res = u16x4{f32_to_bf16(val[0]), f32_to_bf16(val[1]), f32_to_bf16(val[2]), f32_to_bf16(val[3])};
      }
      unsigned short* dst = out_fm ? out + fm_offset(fm_row, fm_col + cb * 16 + 4 * g, out_fm)
                                   : orow + cb * 16 + 4 * g;
      *reinterpret_cast<u16x4*>(dst) = res;
    }
    if (lse_out && g == 0) lse_out[(int64_t)b * R + r] = lse2 * kLn2;
  } else {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const int64_t prow = ((int64_t)unit * splits + split) * kRows + 16 * mb + j;
    // the parts are read once, by another kernel: written non-temporally
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const f32x4 val = o[cb] * scale_out;
      const bf16x4 pv = bf16x4{static_cast<__bf16>(val[0]), static_cast<__bf16>(val[1]),
                               static_cast<__bf16>(val[2]), static_cast<__bf16>(val[3])};
      __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, pv),
                                  reinterpret_cast<uint64_t*>(part_o + prow * C + cb * 16 + 4 * g));
    }
    if (g == 0) __builtin_nontemporal_store(lse2, part_lse + prow);
  }
}

// ---------------------------------------------------------------------------
// Row-block kernel on 32-row blocks (v_mfma_f32_32x32x16_bf16)
// ---------------------------------------------------------------------------
//
// The same workgroup, key split, DMA ring and tile layout as
// verify_attention_mfma, with each wavefront holding 32 query rows instead
// of 16: per 32-key tile a wavefront reads the tile once from LDS for twice
// the rows, and the per-tile VALU work (the maximum across lanes, the
// rescale test, addresses, loop control) is paid once per 32 rows.  The
// instruction's layouts (checked on the MI355X): A and B, lane l holds row /
// column l % 32, k-elements 8 (l / 32) .. + 7; the FP32 result, lane l
// register i holds row 8 (i / 4) + 4 (l / 32) + i % 4 of column l % 32.
//
//   S^T[key, q] = K . Q^T       A = K (lane l: key l % 32, columns 16 s + 8 (l / 32) .. of k-step s)
//                               B = Q^T (lane l: query row l % 32, the same columns)
//   so lane l holds the scores of query l % 32 against keys
//   {8 a + 4 h + m} (h = l / 32, register i = 4 a + m): the maximum of a
//   query is an in-lane maximum of 16 and one exchange with lane l ^ 32.
//   O^T[c, q] += V^T . P^T      per 16-key step kk, B = P^T is registers
//                               8 kk .. 8 kk + 7 of the scores' layout:
//                               k-element 8 h + e is key 16 kk + 4 h + e
//                               (e < 4) or 16 kk + 8 + 4 h + e - 4; A =
//                               V^T, lane l column 32 cb + l % 32 at those
//                               keys, two transposed 4-row reads
template <int C, int MB, bool TREE>
__global__ __launch_bounds__(kKeySets * MB * 64, 1) void verify_attention_m32(
    const int64_t* __restrict__ positions, const int64_t* __restrict__ tree_base, int xcd_map, int groups,
    int splits, int T, int H, int N, int window, int range_from_positions, const unsigned short* __restrict__ k,
    int64_t ksb, int64_t ksn, const unsigned short* __restrict__ v, int64_t vsb, int64_t vsn,
    const unsigned short* __restrict__ q, const uint64_t* __restrict__ ancestors, const float* __restrict__ sink,
    float scale_log2, RowMap rows, OutGate gate, unsigned short* __restrict__ out, int out_fm,
    float* __restrict__ lse_out, unsigned short* __restrict__ part_o, float* __restrict__ part_lse) {
  static_assert(C == 128, "the 32-row kernel is built for head width 128");
  using G = Tile<C>;
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  constexpr int kRows = 32 * MB;
  constexpr int kXC = C / 8;
  constexpr int kQSteps = C / 16;  // k-steps of the QK^T product (32x32x16)
  constexpr int kCB = C / 32;      // 32-wide column blocks of O
  constexpr int DMAW = MB >= 4 ? 4 : (MB >= 2 ? 2 : 1);
  constexpr int kCnt = G::kLoads / DMAW;
  constexpr int kRing = G::kSlots * G::kElems;
  constexpr int kPitch = C + 4;
  static_assert(G::kLoads % DMAW == 0, "DMA split");
  static_assert(MB * (32 * kPitch + 64) * 4 <= kKeySets * kRing * 2, "the merge buffer reuses the rings");
  __shared__ __attribute__((aligned(16))) unsigned short lds[kKeySets * kRing];
  __shared__ __attribute__((aligned(16))) unsigned short qlds[MB * 32 * C];  // each m-block's Q^T operands

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kset = wid / MB, mb = wid % MB;
  const int j = lane & 31;  // this lane's query row (S^T, O^T columns) or key row (K operand)
  const int h = lane >> 5;  // lane half

  // Workgroups are dealt to the 8 XCDs in turn: every group and split of a
  // batch row share one XCD (its L2), where several groups read the same
  // keys and values
  int unit, split;
  {
    const int L = blockIdx.x;
    if (xcd_map) {
      const int slot = L >> 3, per_row = groups * splits;
      const int bb = (L & 7) + 8 * (slot / per_row), rem = slot % per_row;
      unit = bb * groups + rem / splits;
      split = rem % splits;
    } else {
      unit = L / splits;
      split = L % splits;
    }
  }
  const int b = unit / groups;
  const int grp = unit % groups;
  const int R = T * H;
  const int r_base = grp * kRows;
  const QueryPos pos_b = query_pos(positions, tree_base, b, T);

  // The key rows this workgroup's queries can see: the positions come in by
  // one vector load (a lane each), waited for here, before any DMA (the
  // compiler's waits on vector memory cannot count the DMA, so a vector load
  // waited for among the DMA would drain the DMA with it).
  const int r = r_base + 32 * mb + j;
  const bool real = r < R;
  int u_lo = 0, u_hi = N - 1;
  if (range_from_positions)
    union_bounds(pos_b, r_base / H, (min(r_base + kRows, R) - 1) / H, window, N, lane, u_lo, u_hi);
  int s_lo = 0, s_hi = -1;
  if (u_hi >= u_lo) split_range(u_lo, u_hi, splits, split, s_lo, s_hi);
  const int ntiles = s_hi >= s_lo ? (s_hi - s_lo + 1 + 31) / 32 : 0;
  const int niter = (ntiles + kKeySets - 1) / kKeySets;
  const int mine = ntiles > kset ? (ntiles - kset + kKeySets - 1) / kKeySets : 0;

  // DMA of the key/value tiles: as verify_attention_mfma (whole rows per
  // instruction into the swizzled row-major halves).
  const i32x4 krs = buffer_resource(k + (int64_t)b * ksb);
  const i32x4 vrs = buffer_resource(v + (int64_t)b * vsb);
  const uint32_t krow_bytes = (uint32_t)ksn * 2u, vrow_bytes = (uint32_t)vsn * 2u;
  unsigned short* const ring = lds + kset * kRing;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  const bool dma_wave = mb < DMAW;
  const int rbase = row_base(rows, b);
  auto issue = [&](int it) {
    const int tile = kset + it * kKeySets;
    const uint32_t slot = ring_lds + (uint32_t)(it % G::kSlots) * (G::kElems * 2);
#pragma unroll
    for (int c = 0; c < kCnt; ++c) {
      const int ii = mb * kCnt + c;
      const int part = ii / G::kPerHalf, quarter = ii % G::kPerHalf;
      const int row = quarter * (64 / kXC) + lane / kXC;
      const int x = (lane % kXC) ^ (part < 2 ? tile_sigma<C>(row) : v_sigma(row));
      int n = s_lo + tile * 32 + 16 * (part & 1) + row;
      n = n < s_hi ? n : s_hi;
      const uint32_t phys = (uint32_t)(n - rbase) & rows.mask;
      const uint32_t off = phys * (part < 2 ? krow_bytes : vrow_bytes) + 16u * x;
      const uint32_t dst = __builtin_amdgcn_readfirstlane(slot + part * (G::kHalf * 2) + 1024u * quarter);
      i32x4 rs;
#pragma unroll
      for (int e = 0; e < 4; ++e) rs[e] = __builtin_amdgcn_readfirstlane(part < 2 ? krs[e] : vrs[e]);
      // a full-context table read by this query group only: non-temporal (several groups, or the
      // next step's reading of a sliding window, reuse them through the caches)
      if (groups == 1 && window == 0)
        dma_16B_nt(rs, off, dst);
      else
        dma_16B(rs, off, dst);
    }
  };
  // The queries first (each m-block's Q^T operand of k-step s at units
  // 64 s + lane: query row l % 32, columns 16 s + 8 (l / 32) .. + 7), by
  // the first key set; then the first tiles.
  if (kset == 0) {
    i32x4 qrs = buffer_resource(q + (int64_t)b * R * C);
#pragma unroll
    for (int e = 0; e < 4; ++e) qrs[e] = __builtin_amdgcn_readfirstlane(qrs[e]);
    const uint32_t qoff = (uint32_t)(real ? r : R - 1) * (uint32_t)(C * 2) + 16u * h;
    const uint32_t qdst = __builtin_amdgcn_readfirstlane(lds_address(qlds + mb * 32 * C));
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) dma_16B(qrs, qoff + 32u * s, qdst + 1024u * s);
  }
  if (dma_wave) {
#pragma unroll
    for (int it = 0; it < G::kSlots - 1; ++it)
      if (it < mine) issue(it);
  }
  // Per-row bounds: the wavefront's 32 rows span positions t_first..t_last;
  // each position is read with a uniform (scalar) load, on the scalar counter,
  // and the lanes of that position take it.  f_lo, f_hi: the rows every query
  // of the wavefront sees.
  int lo = 0, hi = -1;
  uint64_t anc = 0;
  int f_lo = 0, f_hi = INT_MAX;
  const int64_t tbase = TREE ? tree_base[b] : (int64_t)INT_MAX;
  {
    const int w_first = r_base + 32 * mb;
    if (w_first < R) {
      const int t_first = w_first / H, t_last = (min(w_first + 32, R) - 1) / H;
      const int my_t = real ? r / H : -1;
      for (int t = t_first; t <= t_last; ++t) {
        const Bounds bt = query_bounds(pos_b, t, window, N);
        f_lo = max(f_lo, bt.lo);
        f_hi = min(f_hi, bt.hi);
        if (my_t == t) {
          lo = bt.lo;
          hi = min(bt.hi, s_hi);
        }
        if constexpr (TREE) {
          const uint64_t a = const_load(ancestors, t);
          if (my_t == t) anc = a;
        }
      }
    } else {
      f_hi = -1;
    }
    if (TREE && tbase <= (int64_t)f_hi) f_hi = (int)tbase - 1;
    f_hi = min(f_hi, s_hi);
  }

  bf16x8 qf[kQSteps];
  f32x16 o[kCB];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[cb][i] = 0.f;
  float m_run = kNegInf, l_run = 0.f;
  // K operand of k-step s: key row j (half j / 16, row j % 16), chunk 2 s + h
  const int k_base = (j >> 4) * G::kHalf + 8 * kXC * (j & 15);
  const int k_y = h ^ tile_sigma<C>(j & 15);
  // V^T operand of step kk, column block cb: lane group gq = lane / 16 reads
  // the 4 x 16 block at rows 4 (gq / 2) + rr (+ 8: the second read) of V
  // half 2 + kk, columns 32 cb + 16 (gq % 2) + 4 qq, rr = (lane / 4) % 4, qq = lane % 4
  const int gq = lane >> 4, rr = (lane >> 2) & 3, qq = lane & 3;
  const int va_row = 4 * (gq >> 1) + rr;
  const int va_base = 8 * kXC * va_row + 4 * (qq & 1);
  const int va_y = ((2 * (gq & 1)) | (qq >> 1)) ^ v_sigma(va_row);
  const int vb_base = 8 * kXC * (va_row + 8) + 4 * (qq & 1);
  const int vb_y = ((2 * (gq & 1)) | (qq >> 1)) ^ v_sigma(va_row + 8);

  auto arrive = [&](int t, int later) {
    if (dma_wave && t < mine) {
      if (later >= 2)
        wait_vmcnt<2 * kCnt>();
      else if (later == 1)
        wait_vmcnt<kCnt>();
      else
        wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto qk = [&](int t, f32x16& sc) {
    const unsigned short* st = ring + (t % G::kSlots) * G::kElems;
    // every K fragment requested before the first product
    bf16x8 kf[kQSteps];
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) kf[s] = *reinterpret_cast<const bf16x8*>(st + k_base + 8 * ((2 * s) ^ k_y));
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
    for (int s = 0; s < kQSteps; ++s) sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s], qf[s], sc, 0, 0, 0);
  };
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  auto accumulate = [&](int t, f32x16& sc) {  // the scores masked in place (no copy)
    const unsigned short* st = ring + (t % G::kSlots) * G::kElems;
    const int n0 = s_lo + (kset + t * kKeySets) * 32;
    // the V^T operands requested before the softmax, whose arithmetic covers their latency
    s16x8 vt[2][kCB];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const unsigned short* vh = st + (2 + kk) * G::kHalf;
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vh + va_base + 8 * ((4 * cb) ^ va_y)));
        const s16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vh + vb_base + 8 * ((4 * cb) ^ vb_y)));
        vt[kk][cb] = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
    if (!(n0 >= f_lo && n0 + 31 <= f_hi)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int n = n0 + 8 * (i >> 2) + 4 * h + (i & 3);
        bool vis = n >= lo && n <= hi;
        if constexpr (TREE) vis = vis && tree_visible(n, tbase, anc);
        sc[i] = vis ? sc[i] : kNegInf;
      }
    }
    const f32x16& x = sc;
    float mx = score_max(score_max(score_max(x[0], x[1]), score_max(x[2], x[3])),
                         score_max(score_max(x[4], x[5]), score_max(x[6], x[7])));
    mx = score_max(mx, score_max(score_max(score_max(x[8], x[9]), score_max(x[10], x[11])),
                                 score_max(score_max(x[12], x[13]), score_max(x[14], x[15]))));
    {
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = score_max(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const float bm = mx * scale_log2;
    const bool grow = bm > m_run + kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow && m_run != kNegInf)) {
      const float alpha = (grow && m_run != kNegInf) ? __builtin_amdgcn_exp2f(m_run - bm) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) o[cb] *= alpha;
    }
    m_run = grow ? bm : m_run;
    const float neg_m = m_run == kNegInf ? 0.f : -m_run;
    float p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(x[i], scale_log2, neg_m));
    l_run += (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]))) +
             (((p[8] + p[9]) + (p[10] + p[11])) + ((p[12] + p[13]) + (p[14] + p[15])));
    bf16x8 pt[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) pt[kk][e] = static_cast<__bf16>(p[8 * kk + e]);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
        o[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vt[kk][cb]), pt[kk], o[cb], 0, 0,
                                                        0);
  };

  f32x16 s0, sn;
#pragma unroll
  for (int i = 0; i < 16; ++i) s0[i] = sn[i] = 0.f;
  if (kset == 0 && !(dma_wave && mine > 0)) wait_vmcnt<0>();
  arrive(0, min(G::kSlots - 2, mine - 1));  // tile 0 and every m-block's queries are in LDS
#pragma unroll
  for (int s = 0; s < kQSteps; ++s)
    qf[s] = *reinterpret_cast<const bf16x8*>(qlds + mb * 32 * C + 512 * s + 8 * lane);
  if (mine > 0) qk(0, s0);
  auto iteration = [&](int it, f32x16& cur, f32x16& nxt) {
    arrive(it + 1, min(1, mine - 2 - it));
    if (dma_wave && it + G::kSlots - 1 < mine) issue(it + G::kSlots - 1);
    if (it + 1 < mine) qk(it + 1, nxt);
    if (it < mine) accumulate(it, cur);
  };
#pragma unroll 1
  for (int it = 0; it < niter; it += 2) {
    iteration(it, s0, sn);
    if (it + 1 < niter) iteration(it + 1, sn, s0);
  }
  wait_vmcnt<0>();
  {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    l_run = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }

  // ---- merge the key sets (the merge buffer reuses the rings) ----
  __syncthreads();
  float* mbuf = reinterpret_cast<float*>(lds) + mb * (32 * kPitch + 64);  // this m-block's O (row q: 32 cb + c), m, l
  if (kset == 1) {
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<f32x4*>(mbuf + j * kPitch + 32 * cb + 8 * a + 4 * h) =
            f32x4{o[cb][4 * a], o[cb][4 * a + 1], o[cb][4 * a + 2], o[cb][4 * a + 3]};
    if (h == 0) {
      mbuf[32 * kPitch + j] = m_run;
      mbuf[32 * kPitch + 32 + j] = l_run;
    }
  }
  __syncthreads();
  if (kset != 0) return;
  {
    const float m1 = mbuf[32 * kPitch + j], l1 = mbuf[32 * kPitch + 32 + j];
    const float M = fmaxf(m_run, m1);
    const float a0 = m_run == kNegInf ? 0.f : exp2f(m_run - M);
    const float a1 = m1 == kNegInf ? 0.f : exp2f(m1 - M);
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const f32x4 w = *reinterpret_cast<const f32x4*>(mbuf + j * kPitch + 32 * cb + 8 * a + 4 * h);
#pragma unroll
        for (int m = 0; m < 4; ++m) o[cb][4 * a + m] = o[cb][4 * a + m] * a0 + w[m] * a1;
      }
    l_run = l_run * a0 + l1 * a1;
    m_run = M;
  }
  if (!real) return;

  float M = m_run, L = l_run, f = 1.f;
  if (splits == 1 && sink) {
    const float sl = sink[r % H] * kLog2e;
    const float M2 = fmaxf(M, sl);
    f = (M == kNegInf) ? 0.f : exp2f(M - M2);
    L = L * f + exp2f(sl - M2);
    M = M2;
  }
  const float scale_out = L > 0.f ? f / L : 0.f;
  const float lse2 = L > 0.f ? M + log2f(L) : kNegInf;
  typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
  if (splits == 1) {
    unsigned short* orow = out + ((int64_t)b * R + r) * C;
    const unsigned short* grow = gate.row<unsigned short>(b, T, r, H, C);
    const int fm_row = b * T + r / H, fm_col = (r % H) * C;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int c0 = 32 * cb + 8 * a + 4 * h;
        u16x4 res;
        if (grow) {
          const u16x4 gv = *reinterpret_cast<const u16x4*>(grow + c0);
#pragma unroll
          for (int m = 0; m < 4; ++m) res[m] = gated_bf16(o[cb][4 * a + m] * scale_out, gv[m]);
        } else {
#pragma unroll
          for (int m = 0; m < 4; ++m) res[m] = f32_to_bf16(o[cb][4 * a + m] * scale_out);
        }
        unsigned short* dst = out_fm ? out + fm_offset(fm_row, fm_col + c0, out_fm) : orow + c0;
        *reinterpret_cast<u16x4*>(dst) = res;
      }
    if (lse_out && h == 0) lse_out[(int64_t)b * R + r] = lse2 * kLn2;
  } else {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const int64_t prow = ((int64_t)unit * splits + split) * kRows + 32 * mb + j;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int c0 = 32 * cb + 8 * a + 4 * h;
        *reinterpret_cast<bf16x4*>(part_o + prow * C + c0) =
            bf16x4{static_cast<__bf16>(o[cb][4 * a] * scale_out), static_cast<__bf16>(o[cb][4 * a + 1] * scale_out),
                   static_cast<__bf16>(o[cb][4 * a + 2] * scale_out),
                   static_cast<__bf16>(o[cb][4 * a + 3] * scale_out)};
      }
    if (h == 0) part_lse[prow] = lse2;
  }
}

// ---------------------------------------------------------------------------
// Sparse MFMA kernel: chosen rows plus the window (at most 16 heads)
// ---------------------------------------------------------------------------
//
// One workgroup of four wavefronts per (query, split).  The query's rows --
// its chosen rows idx[b, t, :], then its window max(0, p - window + 1) ..
// min(p, N - 1), the reference's concatenation (pytorch_kernels.py:213-217)
// -- are a list; the split takes a contiguous part of it, copies the row
// numbers into LDS and cuts it into 32-row tiles, and wavefront w gathers the
// tiles w, w + 4, ... into its own two-tile LDS ring (each lane of an LDS DMA
// fetches the row its list entry names: the gather costs nothing beyond the
// DMA) and multiplies them with the H <= 16 heads of the query as one MFMA
// block (S^T = K . Q^T, O^T += V^T . P^T, as the row-block kernel).  Its
// tiles are chunk-major: DMA instruction ii fills 16 rows x 64 bytes, the
// 16-byte chunk x of row r at unit 16x + (r ^ 12 (x & 1)), so that each
// lane's row is a list entry.  A missing row (-1, or past the table) is fetched as
// a valid one and masked.  The four wavefronts merge through LDS; the splits
// merge in combine_splits.

constexpr int kSparseWaves = 4;
constexpr int kSparseSlots = 2;     // tiles in each wavefront's ring
constexpr int kSparseList = 4096;   // list entries a split holds

template <int C>
__global__ __launch_bounds__(kSparseWaves * 64, 1) void sparse_attention_mfma(
    const unsigned short* __restrict__ q, const unsigned short* __restrict__ k, int64_t ksb, int64_t ksn,
    const unsigned short* __restrict__ v, int64_t vsb, int64_t vsn, const int64_t* __restrict__ idx, int K,
    const int64_t* __restrict__ positions, int window, const float* __restrict__ sink, int T, int H, int N,
    float scale_log2, int splits, int per_split, int xcd_map, OutGate gate, unsigned short* __restrict__ out,
    float* __restrict__ lse_out, unsigned short* __restrict__ part_o, float* __restrict__ part_lse) {
  using G = Tile<C>;
  constexpr int kWaveRing = kSparseSlots * G::kElems;  // elements of one wavefront's ring
  constexpr int kPitch = C + 4;                        // merge buffer row pitch (floats)
  static_assert(16 * kPitch + 32 <= kWaveRing / 2, "a wavefront's merge buffer fits in its ring");
  __shared__ __attribute__((aligned(16))) unsigned short ring_all[kSparseWaves * kWaveRing];
  __shared__ __attribute__((aligned(16))) int rows_lds[kSparseList];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  // unit = b T + t.  With xcd_map (B a multiple of 8), every workgroup of a
  // batch row lands on one XCD (the dispatcher deals workgroups out to the 8
  // XCDs in turn), so rows that several of its queries chose are read from
  // HBM once and from that XCD's L2 after.
  int unit, split;
  if (xcd_map) {
    const int per_row = T * splits, kk = blockIdx.x >> 3;
    const int bb = (blockIdx.x & 7) + 8 * (kk / per_row), within = kk % per_row;
    unit = bb * T + within / splits;
    split = within % splits;
  } else {
    unit = blockIdx.x / splits;
    split = blockIdx.x % splits;
  }
  const int b = unit / T;
  const int64_t p = positions[unit];
  const int64_t lo64 = p - window + 1;
  const int lo = lo64 > 0 ? (int)lo64 : 0;
  const int hi = p < (int64_t)N - 1 ? (int)p : N - 1;
  const int nwin = hi >= lo ? hi - lo + 1 : 0;
  const int e0 = split * per_split;
  const int cnt = max(0, min(K + nwin, e0 + per_split) - e0);
  // Q^T operand: head j of the query (a padding head repeats head H - 1),
  // loaded with the row list and waited for before the first DMA (the
  // compiler's waits on vector memory cannot count the DMA, so a load waited
  // for among the DMA would drain the DMA with it)
  bf16x8 qf[G::kSteps];
  {
    const unsigned short* qrow = q + ((int64_t)unit * H + min(j, H - 1)) * C;
#pragma unroll
    for (int s = 0; s < G::kSteps; ++s) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * g);
  }
  for (int i = threadIdx.x; i < per_split; i += kSparseWaves * 64) {
    const int e = e0 + i;
    int n = -1;
    if (i < cnt) {
      if (e < K) {
        const int64_t chosen = idx[(int64_t)unit * K + e];
        n = chosen >= 0 && chosen < N ? (int)chosen : -1;
      } else {
        n = lo + (e - K);
      }
    }
    rows_lds[i] = n;
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < G::kSteps; ++s) asm volatile("" ::"v"(qf[s]));
  const int ntiles = (cnt + 31) / 32;
  const int mine = ntiles > w ? (ntiles - w + kSparseWaves - 1) / kSparseWaves : 0;  // tiles w, w + 4, ...
  const int fallback = nwin > 0 ? lo : 0;  // a valid row for a missing entry's DMA

  const i32x4 krs = buffer_resource(k + (int64_t)b * ksb);
  const i32x4 vrs = buffer_resource(v + (int64_t)b * vsb);
  const uint32_t krow_bytes = (uint32_t)ksn * 2u, vrow_bytes = (uint32_t)vsn * 2u;
  unsigned short* const ring = ring_all + w * kWaveRing;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  auto issue = [&](int i) {  // tile w + 4 i into slot i % 2
    const int tile = w + kSparseWaves * i;
    const uint32_t slot = ring_lds + (uint32_t)(i % kSparseSlots) * (G::kElems * 2);
#pragma unroll
    for (int ii = 0; ii < G::kLoads; ++ii) {
      const int part = ii / G::kPerHalf, chunk = ii % G::kPerHalf;
      const int le = tile * 32 + 16 * (part & 1) + (j ^ (12 * (g & 1)));
      int n = le < cnt ? rows_lds[le] : -1;
      n = n < 0 ? fallback : n;
      const uint32_t off = (uint32_t)n * (part < 2 ? krow_bytes : vrow_bytes) + 64u * chunk + 16u * g;
      dma_16B(part < 2 ? krs : vrs, off, slot + part * (G::kHalf * 2) + 1024u * chunk);
    }
  };
  for (int i = 0; i < kSparseSlots; ++i)
    if (i < mine) issue(i);

  const int tr_off =
      128 * ((lane & 3) >> 1) + 8 * ((4 * g + ((lane >> 2) & 3)) ^ (12 * ((lane >> 1) & 1))) + 4 * (lane & 1);
  const int k_off = 128 * g + 8 * (j ^ (12 * (g & 1)));

  f32x4 o[G::kCBlocks];
#pragma unroll
  for (int cb = 0; cb < G::kCBlocks; ++cb) o[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;
#pragma unroll 1
  for (int i = 0; i < mine; ++i) {
    if (i + 1 < mine)
      wait_vmcnt<G::kLoads>();
    else
      wait_vmcnt<0>();
    const unsigned short* st = ring + (i % kSparseSlots) * G::kElems;
    const int tile = w + kSparseWaves * i;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < G::kSteps; ++s) {
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(st + 512 * s + k_off);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(st + G::kHalf + 512 * s + k_off);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[s], s1, 0, 0, 0);
    }
    // keys 4g + i of each half: masked where the entry names no row
    float x[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int le = tile * 32 + 16 * h + 4 * g;
      const int4 ns = *reinterpret_cast<const int4*>(rows_lds + le);  // le + 3 < per_split: a whole tile
      const f32x4 sv = h ? s1 : s0;
      x[4 * h + 0] = le + 0 < cnt && ns.x >= 0 ? sv[0] : kNegInf;
      x[4 * h + 1] = le + 1 < cnt && ns.y >= 0 ? sv[1] : kNegInf;
      x[4 * h + 2] = le + 2 < cnt && ns.z >= 0 ? sv[2] : kNegInf;
      x[4 * h + 3] = le + 3 < cnt && ns.w >= 0 ? sv[3] : kNegInf;
    }
    const float bm = group_max(score_max(score_max(score_max(x[0], x[1]), score_max(x[2], x[3])),
                                         score_max(score_max(x[4], x[5]), score_max(x[6], x[7])))) *
                     scale_log2;
    const bool grow = bm > m_run + kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow && m_run != kNegInf)) {
      const float alpha = (grow && m_run != kNegInf) ? __builtin_amdgcn_exp2f(m_run - bm) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < G::kCBlocks; ++cb) o[cb] *= alpha;
    }
    m_run = grow ? bm : m_run;
    const float neg_m = m_run == kNegInf ? 0.f : -m_run;
    float pr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pr[e] = __builtin_amdgcn_exp2f(fmaf(x[e], scale_log2, neg_m));
    l_run += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
    const bf16x8 pt = pack_bf16x8(pr);
    const unsigned short* vs = st + 2 * G::kHalf + tr_off;
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vs + 256 * cb));
      const s16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vs + G::kHalf + 256 * cb));
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      const s16x8 vt = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
      o[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vt), pt, o[cb], 0, 0, 0);
    }
    // the slot is free once its values have reached the matrix cores
    if (i + kSparseSlots < mine) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(i + kSparseSlots);
    }
  }
  wait_vmcnt<0>();
  l_run = group_sum(l_run);

  // ---- merge the four wavefronts (each one's buffer in its own ring) ----
  float* mine_buf = reinterpret_cast<float*>(ring);
#pragma unroll
  for (int cb = 0; cb < G::kCBlocks; ++cb)
    *reinterpret_cast<f32x4*>(mine_buf + j * kPitch + cb * 16 + 4 * g) = o[cb];
  if (g == 0) {
    mine_buf[16 * kPitch + j] = m_run;
    mine_buf[16 * kPitch + 16 + j] = l_run;
  }
  __syncthreads();
  constexpr int kQuads8 = C / 8;
  const int item = threadIdx.x;
  if (item >= 16 * kQuads8) return;
  const int jr = item / kQuads8, c8 = (item % kQuads8) * 8;
  if (jr >= H) return;
  float M = kNegInf;
#pragma unroll
  for (int ww = 0; ww < kSparseWaves; ++ww)
    M = fmaxf(M, reinterpret_cast<const float*>(ring_all + ww * kWaveRing)[16 * kPitch + jr]);
  float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (M != kNegInf) {
#pragma unroll
    for (int ww = 0; ww < kSparseWaves; ++ww) {
      const float* buf = reinterpret_cast<const float*>(ring_all + ww * kWaveRing);
      const float mw = buf[16 * kPitch + jr];
      if (mw == kNegInf) continue;
      const float a = exp2f(mw - M);
      L += buf[16 * kPitch + 16 + jr] * a;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += buf[jr * kPitch + c8 + e] * a;
    }
  }
  const int r = (unit % T) * H + jr;  // query row within the batch row
  if (splits == 1) {
    float f = 1.f;
    if (sink) {
      const float sl = sink[jr] * kLog2e;
      const float M2 = fmaxf(M, sl);
      f = M == kNegInf ? 0.f : exp2f(M - M2);
      L = L * f + exp2f(sl - M2);
      M = M2;
    }
    const float inv = L > 0.f ? f / L : 0.f;
    const unsigned short* grow = gate.row<unsigned short>(b, T, r, H, C);
    u16x8 res;
#pragma unroll
    for (int e = 0; e < 8; ++e) res[e] = grow ? gated_bf16(acc[e] * inv, grow[c8 + e]) : f32_to_bf16(acc[e] * inv);
    *reinterpret_cast<u16x8*>(out + ((int64_t)unit * H + jr) * C + c8) = res;
    if (lse_out && c8 == 0) lse_out[(int64_t)unit * H + jr] = L > 0.f ? (M + log2f(L)) * kLn2 : kNegInf;
  } else {
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int64_t prow = ((int64_t)unit * splits + split) * H + jr;
    u16x8 res;
#pragma unroll
    for (int e = 0; e < 8; ++e) res[e] = f32_to_bf16(acc[e] * inv);
    *reinterpret_cast<u16x8*>(part_o + prow * C + c8) = res;
    if (c8 == 0) part_lse[prow] = L > 0.f ? M + log2f(L) : kNegInf;
  }
}

// ---------------------------------------------------------------------------
// Key-parallel MFMA kernel (at most 80 query rows, no tree mask)
// ---------------------------------------------------------------------------
//
// One workgroup of four wavefronts (one per SIMD) per (batch row, key split).
// Every wavefront holds all R <= 16 MB query rows of the batch row (Q^T in
// registers, the O^T accumulators of every row) and owns every fourth
// 32-row key tile of the split: it DMAs its tiles into a private LDS ring and
// reads each byte of them once, so the loop has no workgroup barrier and the
// LDS traffic is the key/value bytes themselves.  The four partial softmaxes
// are merged through LDS at the end; each wavefront then finishes a quarter
// of the head columns.
//
// LDS layouts (bank-conflict free for the reads that use them):
//   K and Q rows: the 16-byte chunk q of row r at chunk position q ^ fk(r),
//     so the 16 lanes of a 128-bit operand read (16 rows, one chunk) hit 16
//     distinct 16-byte bank groups;
//   V rows: the 32-byte segment s of row r at segment position s ^ fv(r), so
//     a transposed 64-bit read (8 rows x 32 bytes per half-wavefront) hits
//     distinct 32-byte bank groups.
// The DMA writes 1 KiB of LDS per instruction (lane l at +16 l), so each lane
// fetches the global chunk that belongs at its LDS position.

template <int C>
struct KTile {
  static constexpr int kRowBytes = 2 * C;            // one bf16 key, value or query row
  static constexpr int kLoads = 32 * kRowBytes / 1024;  // DMA instructions per 32 rows of K (or V)
  static constexpr int kRowsPerLoad = 1024 / kRowBytes;
  static constexpr int kChunks = C / 8;              // 16-byte chunks per row
  static constexpr int kSteps = C / 32;              // k-steps of the QK^T product
  static constexpr int kCBlocks = C / 16;            // 16-column blocks of O
  static constexpr int kSlots = C == 64 ? 4 : 2;     // ring depth (tiles) per wavefront
  static constexpr int kSlotBytes = 2 * 32 * kRowBytes;  // K tile then V tile
};
constexpr int kKeyWaves = 4;

template <int C>
__device__ __forceinline__ int swz_k(int r) {
  return (r / (128 / C)) & (C / 8 - 1);
}
template <int C>
__device__ __forceinline__ int swz_v(int r) {
  return (r / (128 / C)) & (C / 16 - 1);
}

// vmcnt wait for a runtime count n in [0, 3 * kLoads]: the tiles still
// allowed in flight behind the one needed.
template <int kPer>
__device__ __forceinline__ void wait_tiles_behind(int tiles) {
  if (tiles >= 3)
    wait_vmcnt<6 * kPer>();
  else if (tiles == 2)
    wait_vmcnt<4 * kPer>();
  else if (tiles == 1)
    wait_vmcnt<2 * kPer>();
  else
    wait_vmcnt<0>();
}

template <int C, int MB, bool TREE>
__global__ __launch_bounds__(kKeyWaves * 64, 1) void verify_attention_keys(
    const unsigned short* __restrict__ q, const unsigned short* __restrict__ k, int64_t ksb, int64_t ksn,
    const unsigned short* __restrict__ v, int64_t vsb, int64_t vsn, const int64_t* __restrict__ positions,
    int window, const int64_t* __restrict__ tree_base, const uint64_t* __restrict__ ancestors,
    const float* __restrict__ sink, int T, int H, int N, float scale_log2, int splits, int xcd_map,
    unsigned short* __restrict__ out, float* __restrict__ lse_out, unsigned short* __restrict__ part_o,
    float* __restrict__ part_lse) {
  using G = KTile<C>;
  constexpr int kRows = 16 * MB;
  constexpr int kQLoads = kRows * G::kRowBytes / 1024;
  constexpr int kOwn = G::kCBlocks / kKeyWaves;  // column blocks each wavefront finishes
  constexpr int kBlockFloats = kRows * 16;       // one column block of O for every row
  constexpr int kPerK = 16 / G::kRowsPerLoad;    // K DMA pieces after which the swizzle repeats
  constexpr int kPerV = G::kRowsPerLoad >= 8 ? 1 : 8 / G::kRowsPerLoad;
  static_assert(G::kLoads <= 16 && 6 * G::kLoads < 64, "vmcnt range");
  static_assert(kOwn >= 1, "head width");
  static_assert(kKeyWaves * (G::kCBlocks - kOwn) * kBlockFloats * 4 + kKeyWaves * kRows * 8 <=
                    kKeyWaves * G::kSlots * G::kSlotBytes,
                "the merge buffers reuse the rings");
  __shared__ __attribute__((aligned(16))) unsigned char ring_all[kKeyWaves * G::kSlots * G::kSlotBytes];
  __shared__ __attribute__((aligned(16))) unsigned char qlds[kRows * G::kRowBytes];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15;
  const int g = lane >> 4;

  int b, split;
  {
    const int L = blockIdx.x;
    if (xcd_map) {  // the splits of one batch row on one XCD (workgroups go round-robin over the 8)
      const int kk = L >> 3;
      b = (L & 7) + 8 * (kk / splits);
      split = kk % splits;
    } else {
      b = L / splits;
      split = L % splits;
    }
  }
  const int R = T * H;
  const QueryPos pos_b = query_pos(positions, tree_base, b, T);
  // DMA lane roles: lane l fills row rr of a piece (kRowsPerLoad whole rows), 16-byte position p.
  const int rr = lane / G::kChunks, p = lane % G::kChunks;

  // Queries first: wavefront w DMAs the 1 KiB pieces w, w + 4, ... of the
  // R rows (padding rows repeat row R - 1).
  {
    i32x4 qrs = buffer_resource(q + (int64_t)b * R * C);
#pragma unroll
    for (int e = 0; e < 4; ++e) qrs[e] = __builtin_amdgcn_readfirstlane(qrs[e]);
    const uint32_t qdst = __builtin_amdgcn_readfirstlane(lds_address(qlds));
#pragma unroll
    for (int ii = 0; ii < kQLoads; ++ii) {
      if (ii % kKeyWaves != w) continue;
      const int row = ii * G::kRowsPerLoad + rr;
      const int src = row < R ? row : R - 1;
      dma_16B(qrs, (uint32_t)src * G::kRowBytes + 16u * (uint32_t)(p ^ swz_k<C>(row)), qdst + 1024u * ii);
    }
  }

  // Per-position bounds through scalar loads: the union u_lo..u_hi of the
  // rows any query sees, the rows f_lo..f_hi every query sees, and for each
  // of this lane's query rows (row 16 mb + j) its own range.
  int u_lo = INT_MAX, u_hi = -1, f_lo = 0, f_hi = INT_MAX;
  int lo[MB], hi[MB];
  int row_t[MB];
  uint64_t anc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = 16 * mb + j;
    row_t[mb] = row < R ? row / H : -1;
    lo[mb] = 0;
    hi[mb] = -1;
    anc[mb] = 0;
  }
  const int64_t tbase = TREE ? tree_base[b] : (int64_t)INT_MAX;
  for (int t = 0; t < T; ++t) {
    const Bounds bt = query_bounds(pos_b, t, window, N);
    f_lo = max(f_lo, bt.lo);
    f_hi = min(f_hi, bt.hi);
    if (bt.hi >= bt.lo) {
      u_lo = min(u_lo, bt.lo);
      u_hi = max(u_hi, bt.hi);
    }
    uint64_t a = 0;
    if constexpr (TREE) a = ancestors[t];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      if (row_t[mb] == t) {
        lo[mb] = bt.lo;
        hi[mb] = bt.hi;
        anc[mb] = a;
      }
  }
  if (TREE && tbase <= (int64_t)f_hi) f_hi = (int)tbase - 1;  // tree nodes are masked per query
  int s_lo = 0, s_hi = -1;
  if (u_hi >= u_lo) {
    const int U = u_hi - u_lo + 1;
    int per = (U + splits - 1) / splits;
    per = (per + 32 * kKeyWaves - 1) / (32 * kKeyWaves) * (32 * kKeyWaves);
    s_lo = u_lo + split * per;
    s_hi = min(s_lo + per - 1, u_hi);
  }
  f_hi = min(f_hi, s_hi);
  const int ntiles = s_hi >= s_lo ? (s_hi - s_lo + 1 + 31) / 32 : 0;
  const int mine = ntiles > w ? (ntiles - w + kKeyWaves - 1) / kKeyWaves : 0;  // tiles w, w + 4, ...

  // This wavefront's ring and its tile DMA: K rows then V rows, kLoads
  // pieces each.  A whole tile inside the split goes with per-lane offsets
  // fixed at the start and the tile's row offset as the scalar offset; the
  // last, partial tile clamps each row to the split (the extra rows are
  // masked).
  unsigned char* const ring = ring_all + w * G::kSlots * G::kSlotBytes;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  const i32x4 krs = buffer_resource(k + (int64_t)b * ksb);
  const i32x4 vrs = buffer_resource(v + (int64_t)b * vsb);
  const uint32_t krow_bytes = (uint32_t)ksn * 2u, vrow_bytes = (uint32_t)vsn * 2u;
  uint32_t kvo[kPerK], vvo[kPerV];
#pragma unroll
  for (int m = 0; m < kPerK; ++m) kvo[m] = (uint32_t)rr * krow_bytes + 16u * (uint32_t)(p ^ swz_k<C>(m * G::kRowsPerLoad + rr));
#pragma unroll
  for (int m = 0; m < kPerV; ++m)
    vvo[m] = (uint32_t)rr * vrow_bytes + 32u * (uint32_t)((p >> 1) ^ swz_v<C>(m * G::kRowsPerLoad + rr)) + 16u * (uint32_t)(p & 1);
  auto issue_k = [&](int i) {
    const uint32_t slot = ring_lds + (uint32_t)(i % G::kSlots) * G::kSlotBytes;
    const int n0 = s_lo + (w + kKeyWaves * i) * 32;
    if (n0 + 31 <= s_hi) {
#pragma unroll
      for (int ii = 0; ii < G::kLoads; ++ii)
        dma_16B_at(krs, kvo[ii % kPerK], (uint32_t)(n0 + ii * G::kRowsPerLoad) * krow_bytes, slot + 1024u * ii);
    } else {
#pragma unroll
      for (int ii = 0; ii < G::kLoads; ++ii) {
        const int tr = ii * G::kRowsPerLoad + rr;
        const int n = min(n0 + tr, s_hi);
        dma_16B(krs, (uint32_t)n * krow_bytes + 16u * (uint32_t)(p ^ swz_k<C>(tr)), slot + 1024u * ii);
      }
    }
  };
  auto issue_v = [&](int i) {
    const uint32_t slot = ring_lds + (uint32_t)(i % G::kSlots) * G::kSlotBytes + 32u * G::kRowBytes;
    const int n0 = s_lo + (w + kKeyWaves * i) * 32;
    if (n0 + 31 <= s_hi) {
#pragma unroll
      for (int ii = 0; ii < G::kLoads; ++ii)
        dma_16B_at(vrs, vvo[ii % kPerV], (uint32_t)(n0 + ii * G::kRowsPerLoad) * vrow_bytes, slot + 1024u * ii);
    } else {
#pragma unroll
      for (int ii = 0; ii < G::kLoads; ++ii) {
        const int tr = ii * G::kRowsPerLoad + rr;
        const int n = min(n0 + tr, s_hi);
        const int seg = (p >> 1) ^ swz_v<C>(tr);
        dma_16B(vrs, (uint32_t)n * vrow_bytes + 32u * (uint32_t)seg + 16u * (uint32_t)(p & 1), slot + 1024u * ii);
      }
    }
  };
#pragma unroll
  for (int i = 0; i < G::kSlots; ++i)
    if (i < mine) {
      issue_k(i);
      issue_v(i);
    }

  // Queries: every wavefront's share is in LDS once each has waited for its
  // own (everything but its tiles) and the workgroup has met.
  wait_tiles_behind<G::kLoads>(min(mine, G::kSlots));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // Per-lane LDS offsets.  K operand of k-step s (and Q^T, with the query
  // rows): row j, chunk 4 s + g.  Transposed V read of column block cb: lane
  // 16 g + 4 y + qq addresses row 4 g + y, columns 16 cb + 4 qq .. + 3 (the
  // second read adds 16 rows; the swizzles repeat every 16 rows).
  uint32_t ko[G::kSteps], vo[G::kCBlocks];
#pragma unroll
  for (int s = 0; s < G::kSteps; ++s) ko[s] = (uint32_t)(j * G::kRowBytes + 16 * ((4 * s + g) ^ swz_k<C>(j)));
  {
    const int vy = 4 * g + ((lane >> 2) & 3), vqq = lane & 3;
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb)
      vo[cb] = (uint32_t)(vy * G::kRowBytes + 32 * (cb ^ swz_v<C>(vy)) + 8 * vqq);
  }

  f32x4 o[G::kCBlocks][MB];
  float m_run[MB], l_run[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    m_run[mb] = kNegInf;
    l_run[mb] = 0.f;
  }

  // One 32-key tile.  FIRST: the wavefront's first tile, which starts the
  // O^T accumulators (no rescale can be needed: every row's reference
  // maximum is still -inf).
  auto step = [&](int i, auto first_c) {
    constexpr bool FIRST = decltype(first_c)::value;
    wait_tiles_behind<G::kLoads>(min(mine - 1 - i, G::kSlots - 1));
    const unsigned char* st = ring + (i % G::kSlots) * G::kSlotBytes;
    const unsigned char* sv = st + 32 * G::kRowBytes;
    const int n0 = s_lo + (w + kKeyWaves * i) * 32;

    // S^T = K . Q^T for every row block: K is the A operand (lane (j, g)
    // holds key row 16 kb + j, chunk 4 s + g), Q^T the B operand.
    bf16x8 kop[2][G::kSteps];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int s = 0; s < G::kSteps; ++s)
        kop[kb][s] = *reinterpret_cast<const bf16x8*>(st + 16 * kb * G::kRowBytes + ko[s]);
    f32x4 sacc[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int s = 0; s < G::kSteps; ++s) {
        const bf16x8 qs = *reinterpret_cast<const bf16x8*>(qlds + 16 * mb * G::kRowBytes + ko[s]);
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        sacc[mb][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[0][s], qs, s == 0 ? z : sacc[mb][0], 0, 0, 0);
        sacc[mb][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[1][s], qs, s == 0 ? z : sacc[mb][1], 0, 0, 0);
      }
    }
    // The keys of the slot are read: refill them while the softmax runs.
    if (i + G::kSlots < mine) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_k(i + G::kSlots);
    }

    // Row maxima on the raw scores (the scale is positive; lane column j is
    // the query row, lane (j, g) holds keys n0 + 16 kb + 4 g + e).  A row's
    // reference maximum is its first finite tile maximum and moves only when
    // a later one exceeds it by more than 2^kRescaleLog2 (p then stays below
    // 2^32, far inside the fp32 and bf16 range; the result is exact either
    // way).  Moving it from -inf needs no rescale (O and l are still 0); a
    // real rescale is rare and done in one branch for the whole tile.
    const bool full = n0 >= f_lo && n0 + 31 <= f_hi;
    float x[MB][8], tmax[MB];
    bool grow[MB];
    bool rescale = false;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[mb][e] = sacc[mb][0][e];
        x[mb][4 + e] = sacc[mb][1][e];
      }
      if (!full) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int n = n0 + 16 * (e >> 2) + 4 * g + (e & 3);
          bool vis = n >= lo[mb] && n <= hi[mb] && n <= s_hi;
          if constexpr (TREE) vis = vis && tree_visible(n, tbase, anc[mb]);
          x[mb][e] = vis ? x[mb][e] : kNegInf;
        }
      }
      const float* xm = x[mb];
      const float bm =
          group_max(fmaxf(fmaxf(fmaxf(xm[0], xm[1]), fmaxf(xm[2], xm[3])), fmaxf(fmaxf(xm[4], xm[5]), fmaxf(xm[6], xm[7])))) *
          scale_log2;
      tmax[mb] = bm;
      grow[mb] = bm > m_run[mb] + kRescaleLog2;
      if constexpr (!FIRST) rescale = rescale || (grow[mb] && m_run[mb] != kNegInf);
    }
    if constexpr (!FIRST) {
      if (__builtin_amdgcn_ballot_w64(rescale)) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const float alpha =
              (grow[mb] && m_run[mb] != kNegInf) ? __builtin_amdgcn_exp2f(m_run[mb] - tmax[mb]) : 1.f;
          l_run[mb] *= alpha;
#pragma unroll
          for (int cb = 0; cb < G::kCBlocks; ++cb) {
            // the empty asm pins the accumulators in AGPRs up to here, so the
            // compiler copies them to VGPRs inside this branch, not every tile
            f32x4 t = o[cb][mb];
            asm volatile("" : "+a"(t));
            o[cb][mb] = t * alpha;
          }
        }
      }
    }

    // O^T += V^T . P^T: V^T is the A operand (two transposed reads per
    // column block), P^T the B operand, which the S^T accumulator layout
    // already is (k-index 8 g + e = key 4 g + e of the first 16, 16 + 4 g +
    // e - 4 of the second).
    bf16x8 vop[G::kCBlocks];
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(sv + vo[cb]));
      const s16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(sv + 16 * G::kRowBytes + vo[cb]));
      vop[cb] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7));
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      m_run[mb] = grow[mb] ? tmax[mb] : m_run[mb];
      // a row with no visible key so far has every score at -inf: any finite
      // reference gives p = 0
      const float neg_m = m_run[mb] == kNegInf ? 0.f : -m_run[mb];
      float pe[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pe[e] = __builtin_amdgcn_exp2f(fmaf(x[mb][e], scale_log2, neg_m));
      l_run[mb] += ((pe[0] + pe[1]) + (pe[2] + pe[3])) + ((pe[4] + pe[5]) + (pe[6] + pe[7]));
      const bf16x8 pt = pack_bf16x8(pe);
#pragma unroll
      for (int cb = 0; cb < G::kCBlocks; ++cb) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        o[cb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[cb], pt, FIRST ? z : o[cb][mb], 0, 0, 0);
      }
    }
    // The values of the slot are read: refill them.
    if (i + G::kSlots < mine) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue_v(i + G::kSlots);
    }
  };

  if (mine > 0) {
    step(0, std::integral_constant<bool, true>{});
#pragma unroll 1
    for (int i = 1; i < mine; ++i) step(i, std::integral_constant<bool, false>{});
  } else {
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) o[cb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  wait_vmcnt<0>();
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) l_run[mb] = group_sum(l_run[mb]);

  // ---- merge the four wavefronts (the buffers reuse the rings) ----
  __syncthreads();
  float* stats = reinterpret_cast<float*>(ring_all);  // [wave][row]: m, then l
  float* xbuf = stats + kKeyWaves * kRows * 2;        // [column block][slot 0..2][kBlockFloats]
  if (g == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      stats[(w * kRows + 16 * mb + j) * 2] = m_run[mb];
      stats[(w * kRows + 16 * mb + j) * 2 + 1] = l_run[mb];
    }
  }
  __syncthreads();
  float fac[MB], lse2[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = 16 * mb + j;
    float mw[kKeyWaves], lw[kKeyWaves];
    float M = kNegInf;
#pragma unroll
    for (int u = 0; u < kKeyWaves; ++u) {
      mw[u] = stats[(u * kRows + row) * 2];
      lw[u] = stats[(u * kRows + row) * 2 + 1];
      M = fmaxf(M, mw[u]);
    }
    float L = 0.f;
    if (M != kNegInf) {
#pragma unroll
      for (int u = 0; u < kKeyWaves; ++u)
        if (mw[u] != kNegInf) L += lw[u] * exp2f(mw[u] - M);
    }
    // The sink joins the denominator when the split is the whole range.
    if (splits == 1 && sink && row < R) {
      const float sl = sink[row % H] * kLog2e;
      const float M2 = fmaxf(M, sl);
      L = (M == kNegInf ? 0.f : L * exp2f(M - M2)) + exp2f(sl - M2);
      M = M2;
    }
    fac[mb] = (L > 0.f && m_run[mb] != kNegInf) ? exp2f(m_run[mb] - M) / L : 0.f;
    lse2[mb] = L > 0.f ? M + log2f(L) : kNegInf;
  }
  // Column block cb is finished by wavefront cb / kOwn; the other three
  // leave their scaled share in its slots.
#pragma unroll
  for (int cb = 0; cb < G::kCBlocks; ++cb) {
    const int owner = cb / kOwn;
    if (owner == w) continue;
    const int slot = w < owner ? w : w - 1;
    float* dst = xbuf + (cb * (kKeyWaves - 1) + slot) * kBlockFloats;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) *reinterpret_cast<f32x4*>(dst + (64 * mb + lane) * 4) = o[cb][mb] * fac[mb];
  }
  __syncthreads();
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int cb = 0; cb < G::kCBlocks; ++cb) {
    if (cb / kOwn != w) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int row = 16 * mb + j;
      f32x4 acc = o[cb][mb] * fac[mb];
#pragma unroll
      for (int sl = 0; sl < kKeyWaves - 1; ++sl)
        acc += *reinterpret_cast<const f32x4*>(xbuf + (cb * (kKeyWaves - 1) + sl) * kBlockFloats + (64 * mb + lane) * 4);
      if (row >= R) continue;
      const bf16x4 val = {static_cast<__bf16>(acc[0]), static_cast<__bf16>(acc[1]), static_cast<__bf16>(acc[2]),
                          static_cast<__bf16>(acc[3])};
      unsigned short* dst = splits == 1 ? out + ((int64_t)b * R + row) * C
                                        : part_o + (((int64_t)b * splits + split) * kRows + row) * C;
      *reinterpret_cast<bf16x4*>(dst + cb * 16 + 4 * g) = val;
    }
  }
  if (w == 0 && g == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int row = 16 * mb + j;
      if (row >= R) continue;
      if (splits == 1) {
        if (lse_out) lse_out[(int64_t)b * R + row] = lse2[mb] * kLn2;
      } else {
        part_lse[((int64_t)b * splits + split) * kRows + row] = lse2[mb];
      }
    }
  }
}

// Merges the splits of each query row in a kernel of its own: one thread
// per (batch row, query row, 8 columns).
__global__ __launch_bounds__(256) void combine_splits(const unsigned short* __restrict__ part_o,
                                                      const float* __restrict__ part_lse,
                                                      const float* __restrict__ sink, int B, int T, int H, int C,
                                                      int rows_per_group, int groups, int splits, OutGate gate,
                                                      unsigned short* __restrict__ out, int out_fm,
                                                      float* __restrict__ lse_out) {
  const int R = T * H;
  const int per_row = C / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)B * R * per_row) return;
  const int b = (int)(idx / ((int64_t)R * per_row));
  const int rem = (int)(idx % ((int64_t)R * per_row));
  const int r = rem / per_row;
  const int c8 = (rem % per_row) * 8;
  const int grp = r / rows_per_group, rr = r % rows_per_group;
  const int64_t row0 = ((int64_t)(b * groups + grp) * splits) * rows_per_group + rr;  // split 0's part
  const unsigned short* grow = gate.row<unsigned short>(b, T, r, H, C);
  // out_fm > 0: the output [B T, H C] in the fm layout with out_fm row blocks
  unsigned short* dst8 = out_fm ? out + fm_offset(b * T + r / H, (r % H) * C + c8, out_fm)
                                : out + ((int64_t)b * R + r) * C + c8;
  merge_parts(part_o, part_lse, row0, rows_per_group, splits, C, c8, sink ? sink[r % H] * kLog2e : kNegInf, dst8,
              lse_out ? lse_out + (int64_t)b * R + r : nullptr, grow);
}

// ---------------------------------------------------------------------------
// Generic kernel: one wavefront per (b, t, h)
// ---------------------------------------------------------------------------

constexpr int kMaxC = 256;

template <typename T>
__global__ __launch_bounds__(64) void attention_generic(
    const T* __restrict__ q, const T* __restrict__ k, int64_t ksb, int64_t ksn, const T* __restrict__ v,
    int64_t vsb, int64_t vsn, const int64_t* __restrict__ idx, int K, const int64_t* __restrict__ positions,
    int window, const int64_t* __restrict__ tree_base, const uint64_t* __restrict__ ancestors,
    const float* __restrict__ sink, int T_, int H, int C, int N, float scale_log2, RowMap rows, OutGate gate,
    T* __restrict__ out, float* __restrict__ lse_out) {
  const int lane = threadIdx.x;
  const int h = blockIdx.x % H;
  const int t = blockIdx.x / H;
  const int b = blockIdx.y;
  const int64_t row = ((int64_t)b * T_ + t) * H + h;
  const T* qrow = q + row * C;
  const QueryPos pos_b = query_pos(positions, tree_base, b, T_);

  // Rows visited: the chosen rows idx[b, t, :] (K of them, -1 = none), then
  // the rows max(0, p - window + 1) .. min(p, N - 1) (the sparse form's
  // window drops rows outside [0, N) the same way).
  const Bounds bt = query_bounds(pos_b, t, window, N);
  const int lo = bt.lo, hi = bt.hi;
  const int64_t tbase = tree_base ? tree_base[b] : (int64_t)INT_MAX;
  const uint64_t anc = tree_base ? ancestors[t] : 0ull;
  const int n_window = hi >= lo ? hi - lo + 1 : 0;
  const int total = K + n_window;
  const int64_t* idx_row = idx ? idx + ((int64_t)b * T_ + t) * K : nullptr;
  const int rbase = row_base(rows, b);

  float m_run = kNegInf, l_run = 0.f;
  float acc[kMaxC / 64];
  for (int u = 0; u < kMaxC / 64; ++u) acc[u] = 0.f;
  const int per_lane = (C + 63) / 64;

  for (int base = 0; base < total; base += 64) {
    const int e = base + lane;
    int n = -1;
    if (e < total) {
      if (e < K) {
        const int64_t chosen = idx_row[e];
        n = (chosen >= 0 && chosen < N) ? (int)chosen : -1;
      } else {
        n = lo + (e - K);
        if (tree_base && !tree_visible(n, tbase, anc)) n = -1;
      }
    }
    float z = kNegInf;
    if (n >= 0) {
      const T* krow = k + (int64_t)b * ksb + (int64_t)((uint32_t)(n - rbase) & rows.mask) * ksn;
      float dot = 0.f;
      for (int c = 0; c < C; ++c) dot += load_f32(qrow + c) * load_f32(krow + c);
      z = dot * scale_log2;
    }
    const float bm = wave_max(z);
    const float m_new = fmaxf(m_run, bm);
    if (m_new == kNegInf) continue;
    const float alpha = exp2f(m_run - m_new);
    const float pz = (z == kNegInf) ? 0.f : exp2f(z - m_new);
    l_run = l_run * alpha + wave_sum(pz);
    for (int u = 0; u < per_lane; ++u) acc[u] *= alpha;
    m_run = m_new;
    const int count = min(64, total - base);
    for (int i = 0; i < count; ++i) {
      const float pi = __shfl(pz, i, 64);
      const int ni = __shfl(n, i, 64);
      if (ni < 0) continue;
      const T* vrow = v + (int64_t)b * vsb + (int64_t)((uint32_t)(ni - rbase) & rows.mask) * vsn;
      for (int u = 0; u < per_lane; ++u) {
        const int c = lane + 64 * u;
        if (c < C) acc[u] += pi * load_f32(vrow + c);
      }
    }
  }
  float M = m_run, L = l_run, f = 1.f;
  if (sink) {
    const float sl = sink[h] * kLog2e;
    const float M2 = fmaxf(M, sl);
    f = (M == kNegInf) ? 0.f : exp2f(M - M2);
    L = L * f + exp2f(sl - M2);
    M = M2;
  }
  const float inv = L > 0.f ? f / L : 0.f;
  T* orow = out + row * C;
  const T* grow = gate.row<T>(b, T_, t * H + h, H, C);
  for (int u = 0; u < per_lane; ++u) {
    const int c = lane + 64 * u;
    if (c >= C) continue;
    float val = acc[u] * inv;
    if (grow)  // o in the dtype, times sigmoid(gate) in the dtype, rounded again
      val = rounded<T>(val) * rounded<T>(1.f / (1.f + __expf(-load_f32(grow + c))));
    orow[c] = from_f32<T>(val);
  }
  if (lse_out && lane == 0) lse_out[row] = L > 0.f ? (M + log2f(L)) * kLn2 : kNegInf;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

enum Kind { kGeneric = 0, kRowBlocks = 1, kKeySplit = 2, kRowBlocks32 = 3 };

struct Plan {
  Kind kind;
  int mbw;      // 16-row m-blocks per workgroup (row-block kernels) or per wavefront (key-parallel kernel)
  int groups;   // query-row groups per batch row
  int splits;   // key-range parts per batch row
  size_t bytes; // workspace
};

int pick_mbw(int R) {
  // Query rows per workgroup: every row of a decode step in one group when
  // it fits five 16-row blocks (k+1 = 5 positions of 16 heads), else groups
  // of eight blocks (16 wavefronts, 1024 threads), so that a tree's many
  // query rows stream the keys and values as few times as a workgroup can.
  const int blocks = (R + 15) / 16;
  if (blocks <= 1) return 1;
  if (blocks <= 2) return 2;
  if (blocks <= 3) return 3;
  if (blocks <= 5) return 5;
  return 8;
}

int plan(int B, int T, int H, int c, int N, int window, int dtype, int flags, int requested, Plan* out) {
  if (B <= 0 || T <= 0 || H <= 0 || c <= 0 || N <= 0)
    return fail(WPTV_E_INVALID, "verify_attention: B, T, H, c and N must be positive (got %d, %d, %d, %d, %d)", B,
                T, H, c, N);
  if ((long long)T * H > INT_MAX / 2) return fail(WPTV_E_INVALID, "verify_attention: T*H too large");
  if (dtype != WPTV_F32 && dtype != WPTV_BF16)
    return fail(WPTV_E_UNSUPPORTED, "verify_attention: dtype %d is neither fp32 nor bf16", dtype);
  if (c > kMaxC) return fail(WPTV_E_UNSUPPORTED, "verify_attention: head width %d above %d", c, kMaxC);
  Plan p{};
  const bool mfma = dtype == WPTV_BF16 && (c == 64 || c == 128) && !(flags & WPTV_ATTN_FORCE_GENERIC);
  if (!mfma) {
    p.kind = kGeneric;
    p.mbw = 0;
    p.groups = 1;
    p.splits = 1;
    p.bytes = 0;
    *out = p;
    return WPTV_OK;
  }
  const int R = T * H;
  const int blocks = (R + 15) / 16;
  p.kind = (blocks <= 5 && (flags & WPTV_ATTN_KEY_SPLIT)) ? kKeySplit : kRowBlocks;
  // Head width 128 and more than 128 query rows a batch row (a draft tree,
  // a wide reading): the 32-row blocks (measured on the MI355X at batch 16,
  // 8192 prefix rows and 31 nodes of 16 heads: 54 against 61 us); up to 128
  // rows (a verify step's 80) the 16-row blocks (23.7 against 24.6 us at
  // batch 32, 4096 rows).
  if (c == 128 && !(flags & WPTV_ATTN_KEY_SPLIT) && ((flags & WPTV_ATTN_ROWS32) || R > 128)) p.kind = kRowBlocks32;
  if (p.kind == kKeySplit) {
    p.mbw = blocks;
    p.groups = 1;
  } else if (p.kind == kRowBlocks32) {
    // up to four 32-row blocks per key set (eight wavefronts)
    const int b32 = (R + 31) / 32;
    const int m32 = b32 < 4 ? b32 : 4;
    p.mbw = 2 * m32;
    p.groups = (R + 32 * m32 - 1) / (32 * m32);
  } else {
    p.mbw = pick_mbw(R);
    p.groups = (R + 16 * p.mbw - 1) / (16 * p.mbw);
  }
  // Key rows a group reads: the whole table, or the window plus the span of
  // the query positions (T - 1 for consecutive positions).
  long long span = N;
  if (window > 0 && (long long)window + T - 1 < span) span = (long long)window + T - 1;
  // The smallest useful part: one 32-row tile per wavefront (key-parallel
  // kernel) or two per key set (row-block kernels: with one, the key sets'
  // merge and the part write outweigh the shorter stream; measured on the
  // MI355X at batch 8, a 1024-row window: 13.15 us a call at 8 or 12 splits
  // against 13.75 at 17).
  const long long quantum = p.kind == kKeySplit ? 32 * kKeyWaves : 64 * kKeySets;
  int splits = requested;
  if (splits <= 0) {
    const long long cus = compute_units();
    const long long wgs = (long long)B * p.groups;
    // One workgroup per compute unit.
    long long s = (cus + wgs - 1) / wgs;
    const long long max_s = (span + quantum - 1) / quantum;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    splits = (int)s;
  }
  if (splits > 4096) return fail(WPTV_E_INVALID, "verify_attention: splits %d above 4096", splits);
  p.splits = splits;
  if (splits > 1) {
    // parts: bf16 outputs (normalized per part) and fp32 log-sum-exps
    const size_t rows = (size_t)B * p.groups * splits * 16 * p.mbw;
    p.bytes = align_up(rows * c * 2, 256) + align_up(rows * sizeof(float), 256);
  } else {
    p.bytes = 0;
  }
  *out = p;
  return WPTV_OK;
}

template <int C, int MB, bool TREE>
void launch_keys(dim3 grid, hipStream_t stream, const unsigned short* q, const unsigned short* k, int64_t ksb,
                 int64_t ksn, const unsigned short* v, int64_t vsb, int64_t vsn, const int64_t* positions,
                 int window, const int64_t* tree_base, const uint64_t* ancestors, const float* sink, int T, int H,
                 int N, float scale_log2, int splits, int xcd_map, unsigned short* out, float* lse,
                 unsigned short* part_o, float* part_lse) {
  hipLaunchKernelGGL((verify_attention_keys<C, MB, TREE>), grid, dim3(kKeyWaves * 64), 0, stream, q, k, ksb, ksn,
                     v, vsb, vsn, positions, window, tree_base, ancestors, sink, T, H, N, scale_log2, splits,
                     xcd_map, out, lse, part_o, part_lse);
}

template <int C, int MBW, bool TREE>
void launch_mfma(dim3 grid, hipStream_t stream, const unsigned short* q, const unsigned short* k, int64_t ksb,
                 int64_t ksn, const unsigned short* v, int64_t vsb, int64_t vsn, const int64_t* positions,
                 int window, const int64_t* tree_base, const uint64_t* ancestors, const float* sink, int T, int H,
                 int N, float scale_log2, int groups, int splits, int range_from_positions, int xcd_map,
                 RowMap rows, OutGate gate, unsigned short* out, int out_fm, float* lse, unsigned short* part_o,
                 float* part_lse) {
  hipLaunchKernelGGL((verify_attention_mfma<C, MBW, TREE>), grid, dim3(kKeySets * MBW * 64), 0, stream, positions,
                     tree_base, xcd_map, groups, splits, T, H, N, window, range_from_positions, k, ksb, ksn, v, vsb,
                     vsn, q, ancestors, sink, scale_log2, rows, gate, out, out_fm, lse, part_o, part_lse);
}

template <int MB, bool TREE>
void launch_m32(dim3 grid, hipStream_t stream, const unsigned short* q, const unsigned short* k, int64_t ksb,
                int64_t ksn, const unsigned short* v, int64_t vsb, int64_t vsn, const int64_t* positions, int window,
                const int64_t* tree_base, const uint64_t* ancestors, const float* sink, int T, int H, int N,
                float scale_log2, int groups, int splits, int range_from_positions, int xcd_map, RowMap rows,
                OutGate gate, unsigned short* out, int out_fm, float* lse, unsigned short* part_o, float* part_lse) {
  hipLaunchKernelGGL((verify_attention_m32<128, MB, TREE>), grid, dim3(kKeySets * MB * 64), 0, stream, positions,
                     tree_base, xcd_map, groups, splits, T, H, N, window, range_from_positions, k, ksb, ksn, v, vsb,
                     vsn, q, ancestors, sink, scale_log2, rows, gate, out, out_fm, lse, part_o, part_lse);
}

}  // namespace
}  // namespace wptv

using namespace wptv;

extern "C" int wptv_attention_workspace(int B, int T, int H, int c, int N, int window, int dtype, int flags,
                                        int* splits, size_t* bytes) {
  if (!splits || !bytes) return fail(WPTV_E_INVALID, "attention_workspace: null output pointer");
  Plan p;
  int st = plan(B, T, H, c, N, window, dtype, flags, *splits, &p);
  if (st != WPTV_OK) return st;
  *splits = p.splits;
  *bytes = p.bytes;
  return WPTV_OK;
}

namespace {
// Every attention entry point: the table is addressed through `rows`
// (physical rows phys_rows per batch row), the output optionally gated.
int attend(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n, const void* v, int64_t v_stride_b,
           int64_t v_stride_n, int dtype, const int64_t* positions, int window, const int64_t* tree_base,
           const uint64_t* tree_ancestors, const float* sink, int B, int T, int H, int c, int N, float scale,
           int splits, int flags, RowMap rows, int64_t phys_rows, OutGate gate, void* out, float* lse,
           void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!q || !k || !v || !out || !(positions || tree_base))
    return fail(WPTV_E_INVALID, "verify_attention: q, k, v, out and positions (or a tree) must be given");
  if ((tree_base == nullptr) != (tree_ancestors == nullptr))
    return fail(WPTV_E_INVALID, "verify_attention: tree_base and tree_ancestors go together");
  if (k_stride_n < c || v_stride_n < c)
    return fail(WPTV_E_INVALID, "verify_attention: a row stride below the head width");
  Plan p;
  int st = plan(B, T, H, c, N, window, dtype, flags, splits, &p);
  if (st != WPTV_OK) return st;
  const float scale_log2 = scale * kLog2e;
  if (p.kind != kGeneric && !(scale > 0.f && scale < 1e30f)) p.kind = kGeneric, p.splits = 1, p.bytes = 0;  // the MFMA kernels take row maxima on unscaled scores
  if (p.kind != kGeneric) {
    // 32-bit byte offsets within one batch row's table (buffer loads).
    const bool ok_range =
        (double)phys_rows * (double)(k_stride_n > v_stride_n ? k_stride_n : v_stride_n) * 2.0 < 4.0e9;
    const bool ok_align = ok_range && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && (k_stride_b % 8 == 0) &&
                          (k_stride_n % 8 == 0) && (v_stride_b % 8 == 0) && (v_stride_n % 8 == 0);
    if (!ok_align) p.kind = kGeneric, p.splits = 1, p.bytes = 0;
  }
  // the output in the fm layout (the output projection's operand): the MFMA row-block kernel only
  const int out_fm = (flags & WPTV_ATTN_OUT_FM) ? fm_row_blocks(B * T) : 0;
  if (out_fm && p.kind != kRowBlocks && p.kind != kRowBlocks32)
    return fail(WPTV_E_UNSUPPORTED, "verify_attention: the fm output layout needs the bf16 MFMA row-block kernel "
                                    "(head width 64 or 128, aligned operands, no key split)");
  if (p.kind == kGeneric) {
    dim3 grid(T * H, B);
    if (dtype == WPTV_F32)
      hipLaunchKernelGGL(attention_generic<float>, grid, dim3(64), 0, stream, (const float*)q, (const float*)k,
                         k_stride_b, k_stride_n, (const float*)v, v_stride_b, v_stride_n, nullptr, 0, positions,
                         window, tree_base, tree_ancestors, sink, T, H, c, N, scale_log2, rows, gate, (float*)out,
                         lse);
    else
      hipLaunchKernelGGL(attention_generic<unsigned short>, grid, dim3(64), 0, stream, (const unsigned short*)q,
                         (const unsigned short*)k, k_stride_b, k_stride_n, (const unsigned short*)v, v_stride_b,
                         v_stride_n, nullptr, 0, positions, window, tree_base, tree_ancestors, sink, T, H, c, N,
                         scale_log2, rows, gate, (unsigned short*)out, lse);
    return launched("attention_generic");
  }
  if (p.bytes > 0 && (!workspace || workspace_bytes < p.bytes))
    return fail(WPTV_E_INVALID, "verify_attention: workspace of %zu bytes, %zu needed for %d splits",
                workspace_bytes, p.bytes, p.splits);
  const int R = T * H;
  const int rows_per_group = 16 * p.mbw;
  const size_t part_elem = 2;
  void* part_o = nullptr;
  float* part_lse = nullptr;
  if (p.splits > 1) {
    const size_t rows = (size_t)B * p.groups * p.splits * rows_per_group;
    part_o = workspace;
    part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(rows * c * part_elem, 256));
  }
  const int units = B * p.groups;
  dim3 grid(units * p.splits);
  const int xcd_map = units % 8 == 0 ? 1 : 0;
  const auto* qb = static_cast<const unsigned short*>(q);
  const auto* kb = static_cast<const unsigned short*>(k);
  const auto* vb = static_cast<const unsigned short*>(v);
  auto* ob = static_cast<unsigned short*>(out);
  if (p.kind == kKeySplit) {
    auto* po = static_cast<unsigned short*>(part_o);
#define WPTV_LAUNCH(CC, MM)                                                                                       \
  (tree_base ? launch_keys<CC, MM, true> : launch_keys<CC, MM, false>)(                                           \
      grid, stream, qb, kb, k_stride_b, k_stride_n, vb, v_stride_b, v_stride_n, positions, window, tree_base,     \
      tree_ancestors, sink, T, H, N, scale_log2, p.splits, xcd_map, ob, lse, po, part_lse)
    if (c == 128) {
      switch (p.mbw) {
        case 1: WPTV_LAUNCH(128, 1); break;
        case 2: WPTV_LAUNCH(128, 2); break;
        case 3: WPTV_LAUNCH(128, 3); break;
        case 4: WPTV_LAUNCH(128, 4); break;
        default: WPTV_LAUNCH(128, 5); break;
      }
    } else {
      switch (p.mbw) {
        case 1: WPTV_LAUNCH(64, 1); break;
        case 2: WPTV_LAUNCH(64, 2); break;
        case 3: WPTV_LAUNCH(64, 3); break;
        case 4: WPTV_LAUNCH(64, 4); break;
        default: WPTV_LAUNCH(64, 5); break;
      }
    }
#undef WPTV_LAUNCH
    st = launched("verify_attention_keys");
  } else if (p.kind == kRowBlocks32) {
    const int from_positions = (window > 0 || p.groups > 1 || (flags & WPTV_ATTN_RANGE_FROM_POSITIONS)) ? 1 : 0;
    // the kernel's XCD numbering puts batch row b on XCD b mod 8: a batch count that 8 divides
    const int xcd_rows = B % 8 == 0 ? 1 : 0;
    auto* po = static_cast<unsigned short*>(part_o);
#define WPTV_LAUNCH(MM)                                                                                         \
  (tree_base ? launch_m32<MM, true> : launch_m32<MM, false>)(                                                   \
      grid, stream, qb, kb, k_stride_b, k_stride_n, vb, v_stride_b, v_stride_n, positions, window, tree_base,   \
      tree_ancestors, sink, T, H, N, scale_log2, p.groups, p.splits, from_positions, xcd_rows, rows, gate, ob,      \
      out_fm, lse, po, part_lse)
    switch (p.mbw / 2) {
      case 1: WPTV_LAUNCH(1); break;
      case 2: WPTV_LAUNCH(2); break;
      case 3: WPTV_LAUNCH(3); break;
      default: WPTV_LAUNCH(4); break;
    }
#undef WPTV_LAUNCH
    st = launched("verify_attention_m32");
  } else {
    // Full causal attention of a single query group reads the whole table; any
    // other case takes its key range from the positions.
    const int from_positions = (window > 0 || p.groups > 1 || (flags & WPTV_ATTN_RANGE_FROM_POSITIONS)) ? 1 : 0;
    // the kernel's XCD numbering puts batch row b on XCD b mod 8: a batch count that 8 divides
    const int xcd_rows = B % 8 == 0 ? 1 : 0;
    auto* po = static_cast<unsigned short*>(part_o);
#define WPTV_LAUNCH(CC, MM)                                                                                     \
  (tree_base ? launch_mfma<CC, MM, true> : launch_mfma<CC, MM, false>)(                                         \
      grid, stream, qb, kb, k_stride_b, k_stride_n, vb, v_stride_b, v_stride_n, positions, window, tree_base,   \
      tree_ancestors, sink, T, H, N, scale_log2, p.groups, p.splits, from_positions, xcd_rows, rows, gate, ob,      \
      out_fm, lse, po, part_lse)
    if (c == 128) {
      switch (p.mbw) {
        case 1: WPTV_LAUNCH(128, 1); break;
        case 2: WPTV_LAUNCH(128, 2); break;
        case 3: WPTV_LAUNCH(128, 3); break;
        case 4: WPTV_LAUNCH(128, 4); break;
        case 8: WPTV_LAUNCH(128, 8); break;
        default: WPTV_LAUNCH(128, 5); break;
      }
    } else {
      switch (p.mbw) {
        case 1: WPTV_LAUNCH(64, 1); break;
        case 2: WPTV_LAUNCH(64, 2); break;
        case 3: WPTV_LAUNCH(64, 3); break;
        case 4: WPTV_LAUNCH(64, 4); break;
        case 8: WPTV_LAUNCH(64, 8); break;
        default: WPTV_LAUNCH(64, 5); break;
      }
    }
#undef WPTV_LAUNCH
    st = launched("verify_attention_mfma");
  }
  if (st != WPTV_OK || p.splits == 1) return st;
  // 64-thread workgroups when 256-thread ones would leave compute units idle
  const long long items = (long long)B * R * (c / 8);
  const int threads = items >= 256LL * 256 ? 256 : 64;
  dim3 cgrid((unsigned)((items + threads - 1) / threads));
  hipLaunchKernelGGL(combine_splits, cgrid, dim3(threads), 0, stream,
                     static_cast<const unsigned short*>(part_o), part_lse, sink, B, T, H, c, rows_per_group, p.groups,
                     p.splits, gate, ob, out_fm, lse);
  return launched("combine_splits");
}
}  // namespace

extern "C" int wptv_verify_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                     const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                     const int64_t* positions, int window, const int64_t* tree_base,
                                     const uint64_t* tree_ancestors, const float* sink, int B, int T, int H, int c,
                                     int N, float scale, int splits, int flags, void* out, float* lse,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return attend(q, k, k_stride_b, k_stride_n, v, v_stride_b, v_stride_n, dtype, positions, window, tree_base,
                tree_ancestors, sink, B, T, H, c, N, scale, splits, flags, RowMap{nullptr, 0xffffffffu}, N,
                OutGate{nullptr, 0}, out, lse, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// The allocation-free form of wptv_verify_attention: its parts live in a
// file-scope device array instead of a caller's workspace.  Each device that
// loads the library holds one array until the process ends; its address on a
// device is looked up once (hipGetSymbolAddress, that device current) and
// kept.  Every call on a device shares that device's array, so calls that
// overlap on one device (on two streams, or from two threads) race; calls
// ordered on one stream do not.  The parts need no clearing: every part a
// merge reads is written by the same call first.
// ---------------------------------------------------------------------------
namespace wptv {
namespace {
constexpr size_t kScratchBytes = size_t(16) << 20;
constexpr int kScratchDevices = 64;
std::mutex scratch_mutex;
void* scratch_on[kScratchDevices] = {};
}  // namespace
}  // namespace wptv

__device__ __align__(256) unsigned char scratch[wptv::kScratchBytes];

namespace wptv {
namespace {
// The current device's address of `scratch`, looked up on the first call on that device.
int scratch_address(void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(WPTV_E_HIP, "verify_attention_static: hipGetDevice: %s", hipGetErrorString(err));
  if (device < 0 || device >= kScratchDevices)
    return fail(WPTV_E_UNSUPPORTED, "verify_attention_static: device %d beyond the %d this library serves", device,
                kScratchDevices);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_on[device]) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !address)
      return fail(WPTV_E_HIP, "verify_attention_static: hipGetSymbolAddress(scratch) on device %d: %s", device,
                  hipGetErrorString(err));
    scratch_on[device] = address;
  }
  *out = scratch_on[device];
  return WPTV_OK;
}
}  // namespace
}  // namespace wptv

extern "C" int wptv_verify_attention_static(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                            const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                            const int64_t* positions, int window, const int64_t* tree_base,
                                            const uint64_t* tree_ancestors, const float* sink, int B, int T, int H,
                                            int c, int N, float scale, int splits, int flags, void* out, float* lse,
                                            hipStream_t stream) {
  Plan p;
  int st = plan(B, T, H, c, N, window, dtype, flags, splits, &p);
  if (st != WPTV_OK) return st;
  // a split count of the library's choosing steps down until its parts fit
  // the static array (one split needs none)
  while (splits <= 0 && p.bytes > kScratchBytes && p.splits > 1) {
    st = plan(B, T, H, c, N, window, dtype, flags, p.splits - 1, &p);
    if (st != WPTV_OK) return st;
  }
  if (p.bytes > kScratchBytes)
    return fail(WPTV_E_INVALID,
                "verify_attention_static: B=%d T=%d H=%d c=%d in %d splits needs %zu bytes of parts, above the %zu "
                "bytes of its static scratch; call wptv_verify_attention with a workspace",
                B, T, H, c, p.splits, p.bytes, kScratchBytes);
  void* ws = nullptr;
  if (p.bytes > 0) {
    st = scratch_address(&ws);
    if (st != WPTV_OK) return st;
  }
  return attend(q, k, k_stride_b, k_stride_n, v, v_stride_b, v_stride_n, dtype, positions, window, tree_base,
                tree_ancestors, sink, B, T, H, c, N, scale, p.splits, flags, RowMap{nullptr, 0xffffffffu}, N,
                OutGate{nullptr, 0}, out, lse, ws, p.bytes > 0 ? kScratchBytes : 0, stream);
}

extern "C" int wptv_window_attention_workspace(int B, int T, int H, int c, int window, int dtype, int* splits,
                                               size_t* bytes) {
  if (!splits || !bytes) return fail(WPTV_E_INVALID, "window_attention_workspace: null output pointer");
  if (window <= 0) return fail(WPTV_E_INVALID, "window_attention_workspace: window %d must be > 0", window);
  Plan p;
  const int st = plan(B, T, H, c, window + T - 1, window, dtype, 0, *splits, &p);
  if (st != WPTV_OK) return st;
  *splits = p.splits;
  *bytes = p.bytes;
  return WPTV_OK;
}

extern "C" int wptv_window_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                     const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                     const int64_t* positions, const int64_t* row_base, int ring_rows, int window,
                                     const float* sink, const void* gate, int64_t gate_stride, int B, int T, int H,
                                     int c, float scale, int splits, void* out, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
  if (window <= 0) return fail(WPTV_E_INVALID, "window_attention: window %d must be > 0", window);
  if (ring_rows <= 0) return fail(WPTV_E_INVALID, "window_attention: ring_rows %d must be > 0", ring_rows);
  if (row_base == nullptr && (ring_rows & (ring_rows - 1)) != 0)
    return fail(WPTV_E_INVALID, "window_attention: a ring of %d rows is not a power of 2", ring_rows);
  if (row_base == nullptr && ring_rows < window + T - 1)
    return fail(WPTV_E_INVALID, "window_attention: a ring of %d rows holds less than window + T - 1 = %d", ring_rows,
                window + T - 1);
  if (gate && gate_stride < (int64_t)H * c)
    return fail(WPTV_E_INVALID, "window_attention: gate row stride %lld below H*c", (long long)gate_stride);
  // Logical rows: token positions; the upper bound only keeps hi = p.
  const RowMap rows{row_base, row_base ? 0xffffffffu : (uint32_t)(ring_rows - 1)};
  return attend(q, k, k_stride_b, k_stride_n, v, v_stride_b, v_stride_n, dtype, positions, window, nullptr, nullptr,
                sink, B, T, H, c, INT_MAX / 2, scale, splits, WPTV_ATTN_RANGE_FROM_POSITIONS, rows, ring_rows,
                OutGate{gate, gate_stride}, out, nullptr, workspace, workspace_bytes, stream);
}


namespace {
struct SparsePlan {
  bool mfma;
  int splits, per_split;
  size_t bytes;
};

int sparse_plan(int B, int T, int H, int c, int K, int window, int N, int dtype, int requested, SparsePlan* p) {
  if (B <= 0 || T <= 0 || H <= 0 || c <= 0 || K < 0 || window < 0)
    return fail(WPTV_E_INVALID, "sparse_attention: bad shape B=%d T=%d H=%d c=%d K=%d window=%d", B, T, H, c, K,
                window);
  if (dtype != WPTV_F32 && dtype != WPTV_BF16)
    return fail(WPTV_E_UNSUPPORTED, "sparse_attention: dtype %d is neither fp32 nor bf16", dtype);
  if (c > kMaxC) return fail(WPTV_E_UNSUPPORTED, "sparse_attention: head width %d above %d", c, kMaxC);
  p->mfma = dtype == WPTV_BF16 && (c == 64 || c == 128) && H <= 16;
  p->splits = 1;
  p->per_split = 0;
  p->bytes = 0;
  if (!p->mfma) return WPTV_OK;
  const long long total = (long long)K + (window < N ? window : N);  // the longest list of a query
  long long s = requested;
  if (s <= 0) {
    s = (compute_units() + (long long)B * T - 1) / ((long long)B * T);  // a workgroup per compute unit
    const long long most = (total + 127) / 128;  // at least one tile per wavefront
    if (s > most) s = most;
  }
  const long long least = (total + kSparseList - 1) / kSparseList;  // the list of a split fits its LDS
  if (s < least) s = least;
  if (s < 1) s = 1;
  if (s > 4096) return fail(WPTV_E_INVALID, "sparse_attention: splits %lld above 4096", s);
  long long per = (total + s - 1) / s;
  per = (per + 31) / 32 * 32;
  if (per > kSparseList) return fail(WPTV_E_INVALID, "sparse_attention: %lld rows per split above %d", per, kSparseList);
  p->splits = (int)s;
  p->per_split = (int)(per > 0 ? per : 32);
  if (s > 1) {
    const size_t rows = (size_t)B * T * s * H;
    p->bytes = align_up(rows * c * 2, 256) + align_up(rows * sizeof(float), 256);
  }
  return WPTV_OK;
}
}  // namespace

extern "C" int wptv_sparse_attention_workspace(int B, int T, int H, int c, int K, int window, int N, int dtype,
                                               int* splits, size_t* bytes) {
  if (!splits || !bytes) return fail(WPTV_E_INVALID, "sparse_attention_workspace: null output pointer");
  if (K == 0 && window > 0)  // the window alone: the row-block kernel (wptv_sparse_attention routes it there)
    return wptv_attention_workspace(B, T, H, c, N, window, dtype, WPTV_ATTN_RANGE_FROM_POSITIONS, splits, bytes);
  SparsePlan p;
  const int st = sparse_plan(B, T, H, c, K, window, N, dtype, *splits, &p);
  if (st != WPTV_OK) return st;
  *splits = p.splits;
  *bytes = p.bytes;
  return WPTV_OK;
}

extern "C" int wptv_sparse_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                     const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                     const int64_t* idx, int K, const int64_t* positions, int window,
                                     const float* sink, const void* gate, int64_t gate_stride, int B, int T, int H,
                                     int c, int N, float scale, int splits, void* out, float* lse, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
  if (!q || !k || !v || !positions || !out || (K > 0 && !idx))
    return fail(WPTV_E_INVALID, "sparse_attention: q, k, v, positions, out (and idx when K > 0) must be given");
  if (N <= 0) return fail(WPTV_E_INVALID, "sparse_attention: the table is empty");
  if (k_stride_n < c || v_stride_n < c)
    return fail(WPTV_E_INVALID, "sparse_attention: a row stride below the head width");
  if (gate && gate_stride < (int64_t)H * c)
    return fail(WPTV_E_INVALID, "sparse_attention: gate row stride %lld below H*c", (long long)gate_stride);
  if (K == 0 && window > 0)  // no chosen rows: the window attention of the row-block kernel, reading the window only
    return attend(q, k, k_stride_b, k_stride_n, v, v_stride_b, v_stride_n, dtype, positions, window, nullptr, nullptr,
                  sink, B, T, H, c, N, scale, splits, WPTV_ATTN_RANGE_FROM_POSITIONS, RowMap{nullptr, 0xffffffffu}, N,
                  OutGate{gate, gate_stride}, out, lse, workspace, workspace_bytes, stream);
  SparsePlan p;
  int st = sparse_plan(B, T, H, c, K, window, N, dtype, splits, &p);
  if (st != WPTV_OK) return st;
  const float scale_log2 = scale * kLog2e;
  const bool ok_range = (double)N * (double)(k_stride_n > v_stride_n ? k_stride_n : v_stride_n) * 2.0 < 4.0e9;
  if (p.mfma && !(scale > 0.f && scale < 1e30f && ok_range && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
                  k_stride_b % 8 == 0 && k_stride_n % 8 == 0 && v_stride_b % 8 == 0 && v_stride_n % 8 == 0 &&
                  (!gate || (aligned(gate, 16) && gate_stride % 8 == 0))))
    p.mfma = false;
  const int64_t* rows = K > 0 ? idx : nullptr;
  const OutGate og{gate, gate_stride};
  if (!p.mfma) {
    dim3 grid(T * H, B);
    if (dtype == WPTV_F32)
      hipLaunchKernelGGL(attention_generic<float>, grid, dim3(64), 0, stream, (const float*)q, (const float*)k,
                         k_stride_b, k_stride_n, (const float*)v, v_stride_b, v_stride_n, rows, K, positions, window,
                         nullptr, nullptr, sink, T, H, c, N, scale_log2, RowMap{nullptr, 0xffffffffu}, og,
                         (float*)out, lse);
    else
      hipLaunchKernelGGL(attention_generic<unsigned short>, grid, dim3(64), 0, stream, (const unsigned short*)q,
                         (const unsigned short*)k, k_stride_b, k_stride_n, (const unsigned short*)v, v_stride_b,
                         v_stride_n, rows, K, positions, window, nullptr, nullptr, sink, T, H, c, N, scale_log2,
                         RowMap{nullptr, 0xffffffffu}, og, (unsigned short*)out, lse);
    return launched("attention_generic");
  }
  if (p.bytes > 0 && (!workspace || workspace_bytes < p.bytes))
    return fail(WPTV_E_INVALID, "sparse_attention: workspace of %zu bytes, %zu needed for %d splits", workspace_bytes,
                p.bytes, p.splits);
  unsigned short* part_o = nullptr;
  float* part_lse = nullptr;
  if (p.splits > 1) {
    const size_t rows_n = (size_t)B * T * p.splits * H;
    part_o = static_cast<unsigned short*>(workspace);
    part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(rows_n * c * 2, 256));
  }
  const long long wgs = (long long)B * T * p.splits;
  if (wgs > INT_MAX) return fail(WPTV_E_INVALID, "sparse_attention: grid too large");
  const auto* qb = static_cast<const unsigned short*>(q);
  const auto* kb = static_cast<const unsigned short*>(k);
  const auto* vb = static_cast<const unsigned short*>(v);
  auto* ob = static_cast<unsigned short*>(out);
  if (c == 128)
    hipLaunchKernelGGL(sparse_attention_mfma<128>, dim3((unsigned)wgs), dim3(kSparseWaves * 64), 0, stream, qb, kb,
                       k_stride_b, k_stride_n, vb, v_stride_b, v_stride_n, rows, K, positions, window, sink, T, H, N,
                       scale_log2, p.splits, p.per_split, B % 8 == 0, og, ob, lse, part_o, part_lse);
  else
    hipLaunchKernelGGL(sparse_attention_mfma<64>, dim3((unsigned)wgs), dim3(kSparseWaves * 64), 0, stream, qb, kb,
                       k_stride_b, k_stride_n, vb, v_stride_b, v_stride_n, rows, K, positions, window, sink, T, H, N,
                       scale_log2, p.splits, p.per_split, B % 8 == 0, og, ob, lse, part_o, part_lse);
  st = launched("sparse_attention_mfma");
  if (st != WPTV_OK || p.splits == 1) return st;
  const long long items = (long long)B * T * H * (c / 8);
  dim3 cgrid((unsigned)((items + 255) / 256));
  hipLaunchKernelGGL(combine_splits, cgrid, dim3(256), 0, stream, part_o, part_lse, sink, B, T, H, c, H, T, p.splits,
                     og, ob, 0, lse);
  return launched("combine_splits");
}
