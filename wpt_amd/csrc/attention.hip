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

namespace wptv {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr float kNegInf = -__builtin_inff();

struct Bounds {
  int lo, hi;  // inclusive key-row range a query sees (hi < lo: none)
};

// The key rows query position t of batch row b sees, before the tree mask.
__device__ __forceinline__ Bounds query_bounds(const int64_t* __restrict__ pos_b, int t, int window, int N) {
  const int64_t p = pos_b[t];
  int64_t hi = p < (int64_t)N - 1 ? p : (int64_t)N - 1;
  int64_t lo = window > 0 ? p - window + 1 : 0;
  if (lo < 0) lo = 0;
  Bounds r;
  r.lo = (int)lo;
  r.hi = hi < lo ? (int)lo - 1 : (int)hi;
  return r;
}

__device__ __forceinline__ bool tree_visible(int n, int64_t tbase, uint64_t anc) {
  if ((int64_t)n < tbase) return true;
  const int64_t node = (int64_t)n - tbase;
  return node < 64 && ((anc >> node) & 1ull);
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

// Softmax rescaling is deferred until a row's maximum grows by more than this
// many powers of two (the stale maximum stays the reference for p and l, so
// the result is exact; p stays below 2^8).
constexpr float kRescale = 8.f;

// s_waitcnt with vmcnt = n and the other counters left alone (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
  asm volatile("" ::: "memory");
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// A raw buffer resource over 4 GiB from `base` (gfx9 dword3 format).
__device__ __forceinline__ i32x4 buffer_resource(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = static_cast<int>(static_cast<uint32_t>(a));
  r[1] = static_cast<int>(static_cast<uint32_t>(a >> 32));  // stride 0
  r[2] = -1;
  r[3] = 0x00020000;
  return r;
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// Global -> LDS copy of 16 bytes per lane: lane l's bytes land at LDS byte
// address `lds` + 16 l.  Written as inline assembly so that the compiler's
// conservative wait (all loads, before any LDS read of the kernel) is not
// inserted: the kernel waits for each tile itself.  The s_nop covers the
// M0-write -> LDS-DMA hazard.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_16B(i32x4 rsrc, uint32_t voffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ bf16x8 pack_bf16x8(const float (&p)[8]) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = static_cast<__bf16>(p[e]);
  return r;
}

// max / sum over the four 16-lane groups (lanes j, j+16, j+32, j+48).
__device__ __forceinline__ float group_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
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
// them; a workgroup barrier per iteration hands them over.
template <int C, int MB, bool TREE>
__global__ __launch_bounds__(kKeySets * MB * 64, 1) void verify_attention_mfma(
    const unsigned short* __restrict__ q, const unsigned short* __restrict__ k, int64_t ksb, int64_t ksn,
    const unsigned short* __restrict__ v, int64_t vsb, int64_t vsn, const int64_t* __restrict__ positions,
    int window, const int64_t* __restrict__ tree_base, const uint64_t* __restrict__ ancestors,
    const float* __restrict__ sink, int T, int H, int N, float scale_log2, int groups, int splits,
    int range_from_positions, int xcd_map, unsigned short* __restrict__ out, float* __restrict__ lse_out,
    float* __restrict__ part_o, float* __restrict__ part_lse) {
  using G = Tile<C>;
  constexpr int kRows = 16 * MB;
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

  int unit, split;
  {
    const int L = blockIdx.x;
    if (xcd_map) {
      const int kk = L >> 3;
      unit = (L & 7) + 8 * (kk / splits);
      split = kk % splits;
    } else {
      unit = L / splits;
      split = L % splits;
    }
  }
  const int b = unit / groups;
  const int grp = unit % groups;
  const int R = T * H;
  const int r_base = grp * kRows;
  const int64_t* pos_b = positions + (int64_t)b * T;

  // The key rows this workgroup's queries can see.
  int u_lo = 0, u_hi = N - 1;
  if (range_from_positions) {
    u_lo = INT_MAX;
    u_hi = -1;
    const int t_first = r_base / H, t_last = (min(r_base + kRows, R) - 1) / H;
    for (int t = t_first; t <= t_last; ++t) {
      const Bounds bt = query_bounds(pos_b, t, window, N);
      if (bt.hi >= bt.lo) {
        u_lo = min(u_lo, bt.lo);
        u_hi = max(u_hi, bt.hi);
      }
    }
  }
  int s_lo = 0, s_hi = -1;
  if (u_hi >= u_lo) {
    const int U = u_hi - u_lo + 1;
    int per = (U + splits - 1) / splits;
    per = (per + 32 * kKeySets - 1) / (32 * kKeySets) * (32 * kKeySets);
    s_lo = u_lo + split * per;
    s_hi = min(s_lo + per - 1, u_hi);
  }
  const int ntiles = s_hi >= s_lo ? (s_hi - s_lo + 1 + 31) / 32 : 0;
  const int niter = (ntiles + kKeySets - 1) / kKeySets;       // workgroup iterations
  const int mine = ntiles > kset ? (ntiles - kset + kKeySets - 1) / kKeySets : 0;  // tiles of this key set

  // DMA: instruction ii of a tile covers 16 rows x 64 bytes of one half
  // (part = ii / kPerHalf: K rows 0-15, K rows 16-31, V rows 0-15, V rows 16-31).
  // LDS layout of a half, chunk-major: the 16-byte chunk x of row r at unit
  // 16x + r, so lane l of the instruction fills unit 64 (ii % kPerHalf) + l.
  const i32x4 krs = buffer_resource(k + (int64_t)b * ksb);
  const i32x4 vrs = buffer_resource(v + (int64_t)b * vsb);
  const uint32_t krow_bytes = (uint32_t)ksn * 2u, vrow_bytes = (uint32_t)vsn * 2u;
  unsigned short* const ring = lds + kset * kRing;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  const bool dma_wave = mb < DMAW;
  auto issue = [&](int it) {  // this wavefront's share of the key set's tile of iteration it
    const int tile = kset + it * kKeySets;
    const uint32_t slot = ring_lds + (uint32_t)(it % G::kSlots) * (G::kElems * 2);
#pragma unroll
    for (int c = 0; c < kCnt; ++c) {
      const int ii = mb * kCnt + c;
      const int part = ii / G::kPerHalf, chunk = ii % G::kPerHalf;
      int n = s_lo + tile * 32 + 16 * (part & 1) + j;
      n = n < s_hi ? n : s_hi;  // rows past the split are masked; read a valid one
      const uint32_t off = (uint32_t)n * (part < 2 ? krow_bytes : vrow_bytes) + 64u * chunk + 16u * g;
      dma_16B(part < 2 ? krs : vrs, off, slot + part * (G::kHalf * 2) + 1024u * chunk);
    }
  };
  // The queries go out first (DMA into qlds, each m-block laid out like a
  // key half, so that the Q^T operand of k-step s is unit 64s + lane; the
  // first key set loads them, the second reads them after the first
  // barrier), then the first tiles.  Waiting for tile 0 then implies the
  // queries.  The bounds come through scalar loads, on their own counter, so
  // the compiler needs no vector-memory wait of its own inside the loop (it
  // cannot count the DMA).
  const int r = r_base + 16 * mb + j;
  const bool real = r < R;
  if (kset == 0) {
    const i32x4 qrs = buffer_resource(q + (int64_t)b * R * C);
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
  // each position is read with a uniform (scalar) load and the lanes of that
  // position take it.  f_lo, f_hi: the rows every query of the wavefront sees.
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
          const uint64_t a = ancestors[t];
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
  // per-lane element offset of the transposed V reads: lane 16g + 4rr + qq
  // addresses row 4g + rr, columns 4qq..4qq+3 of a 16-column block
  const int tr_off = 128 * ((lane & 3) >> 1) + 32 * g + 8 * ((lane >> 2) & 3) + 4 * (lane & 1);

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
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(st + 512 * s + 8 * lane);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(st + G::kHalf + 512 * s + 8 * lane);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[s], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[s], s1, 0, 0, 0);
    }
  };
  // The probabilities of a tile against the running maximum, and O^T += V^T . P^T.
  auto accumulate = [&](int t, const f32x4& s0, const f32x4& s1) {
    const unsigned short* st = ring + (t % G::kSlots) * G::kElems;
    const int n0 = s_lo + (kset + t * kKeySets) * 32;
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = s0[i] * scale_log2;
      x[4 + i] = s1[i] * scale_log2;
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
    float bm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    bm = group_max(bm);
    if (bm > m_run + kRescale) {  // this lane's row: rescale its sums to the new maximum
      const float alpha = m_run == kNegInf ? 0.f : __builtin_amdgcn_exp2f(m_run - bm);
      m_run = bm;
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < G::kCBlocks; ++cb) o[cb] *= alpha;
    }
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(x[e] - m_run);  // 0 at -inf; m_run finite here
    if (m_run == kNegInf) {
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = 0.f;
    }
    l_run += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    // P^T operand: lane (j, g) holds k-index 8g + e = key 4g + e of the first
    // half (e < 4), key 16 + 4g + e - 4 of the second; the V^T operand holds
    // the same keys at column cb*16 + j, two transposed 4-row reads.
    const bf16x8 pt = pack_bf16x8(p);
    const unsigned short* vs = st + 2 * G::kHalf + tr_off;
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vs + 256 * cb));
      const s16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vs + G::kHalf + 256 * cb));
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
#pragma unroll 1
  for (int it = 0; it < niter; ++it) {
    arrive(it + 1, min(1, mine - 2 - it));  // every wavefront is done with iteration it - 1
    if (dma_wave && it + G::kSlots - 1 < mine) issue(it + G::kSlots - 1);
    f32x4 n0v = {0.f, 0.f, 0.f, 0.f}, n1v = {0.f, 0.f, 0.f, 0.f};
    if (it + 1 < mine) qk(it + 1, n0v, n1v);
    if (it < mine) accumulate(it, s0, s1);
    s0 = n0v;
    s1 = n1v;
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
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb) {
      const f32x4 val = o[cb] * scale_out;
      *reinterpret_cast<u16x4*>(orow + cb * 16 + 4 * g) =
          u16x4{f32_to_bf16(val[0]), f32_to_bf16(val[1]), f32_to_bf16(val[2]), f32_to_bf16(val[3])};
    }
    if (lse_out && g == 0) lse_out[(int64_t)b * R + r] = lse2 * kLn2;
  } else {
    const int64_t prow = ((int64_t)unit * splits + split) * kRows + 16 * mb + j;
#pragma unroll
    for (int cb = 0; cb < G::kCBlocks; ++cb)
      *reinterpret_cast<f32x4*>(part_o + prow * C + cb * 16 + 4 * g) = o[cb] * scale_out;
    if (g == 0) part_lse[prow] = lse2;
  }
}

// Merges the splits of each query row: fixed order, log-sum-exp weights,
// the sink joining the denominator.  One thread per (batch row, query row,
// 4 columns); the parts of one row are read with independent loads.
template <typename OutT>
__global__ __launch_bounds__(256) void combine_splits(const float* __restrict__ part_o,
                                                       const float* __restrict__ part_lse,
                                                       const float* __restrict__ sink, int B, int R, int H, int C,
                                                       int rows_per_group, int groups, int splits,
                                                       OutT* __restrict__ out, float* __restrict__ lse_out) {
  const int per_row = C / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)B * R * per_row) return;
  const int b = (int)(idx / ((int64_t)R * per_row));
  const int rem = (int)(idx % ((int64_t)R * per_row));
  const int r = rem / per_row;
  const int c4 = (rem % per_row) * 4;
  const int grp = r / rows_per_group, rr = r % rows_per_group;
  const int64_t row0 = ((int64_t)(b * groups + grp) * splits) * rows_per_group + rr;  // split 0's part
  constexpr int kUnroll = 8;
  float M = kNegInf;
  for (int s0 = 0; s0 < splits; s0 += kUnroll) {
    float ls[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) ls[u] = s0 + u < splits ? part_lse[row0 + (int64_t)(s0 + u) * rows_per_group] : kNegInf;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) M = fmaxf(M, ls[u]);
  }
  const float sl = sink ? sink[r % H] * kLog2e : kNegInf;
  const float M2 = fmaxf(M, sl);
  float L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (M2 != kNegInf) {
    for (int s0 = 0; s0 < splits; s0 += kUnroll) {
      float ls[kUnroll];
      f32x4 po[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t prow = row0 + (int64_t)(s0 + u) * rows_per_group;
        const bool in = s0 + u < splits;
        ls[u] = in ? part_lse[prow] : kNegInf;
        po[u] = in ? *reinterpret_cast<const f32x4*>(part_o + prow * C + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (ls[u] == kNegInf) continue;
        const float w = exp2f(ls[u] - M2);
        L += w;
        acc += w * po[u];
      }
    }
    if (sink) L += exp2f(sl - M2);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  OutT* dst = out + ((int64_t)b * R + r) * C + c4;
  for (int e = 0; e < 4; ++e) dst[e] = from_f32<OutT>(acc[e] * inv);
  if (lse_out && c4 == 0) lse_out[(int64_t)b * R + r] = L > 0.f ? (M2 + log2f(L)) * kLn2 : kNegInf;
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
    const float* __restrict__ sink, int T_, int H, int C, int N, float scale_log2, T* __restrict__ out,
    float* __restrict__ lse_out) {
  const int lane = threadIdx.x;
  const int h = blockIdx.x % H;
  const int t = blockIdx.x / H;
  const int b = blockIdx.y;
  const int64_t row = ((int64_t)b * T_ + t) * H + h;
  const T* qrow = q + row * C;
  const int64_t* pos_b = positions + (int64_t)b * T_;

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
      const T* krow = k + (int64_t)b * ksb + (int64_t)n * ksn;
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
      const T* vrow = v + (int64_t)b * vsb + (int64_t)ni * vsn;
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
  for (int u = 0; u < per_lane; ++u) {
    const int c = lane + 64 * u;
    if (c < C) orow[c] = from_f32<T>(acc[u] * inv);
  }
  if (lse_out && lane == 0) lse_out[row] = L > 0.f ? (M + log2f(L)) * kLn2 : kNegInf;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

struct Plan {
  bool mfma;
  int mbw;      // m-blocks per workgroup
  int groups;   // query-row groups per batch row
  int splits;   // key-range parts per batch row
  size_t bytes; // workspace
};

int pick_mbw(int R) {
  // Query rows per workgroup: every row of a decode step in one group when
  // it fits five 16-row blocks (k+1 = 5 positions of 16 heads), else groups
  // of four blocks.
  const int blocks = (R + 15) / 16;
  if (blocks <= 1) return 1;
  if (blocks <= 2) return 2;
  if (blocks <= 3) return 3;
  if (blocks <= 5) return 5;
  return 4;
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
  p.mfma = dtype == WPTV_BF16 && (c == 64 || c == 128) && !(flags & WPTV_ATTN_FORCE_GENERIC);
  if (!p.mfma) {
    p.mbw = 0;
    p.groups = 1;
    p.splits = 1;
    p.bytes = 0;
    *out = p;
    return WPTV_OK;
  }
  const int R = T * H;
  p.mbw = pick_mbw(R);
  p.groups = (R + 16 * p.mbw - 1) / (16 * p.mbw);
  // Key rows a group reads: the whole table, or the window plus the span of
  // the query positions (T - 1 for consecutive positions).
  long long span = N;
  if (window > 0 && (long long)window + T - 1 < span) span = (long long)window + T - 1;
  int splits = requested;
  if (splits <= 0) {
    const long long cus = compute_units();
    const long long wgs = (long long)B * p.groups;
    // Enough workgroups to fill the GPU, each at least one 32-row tile per key set.
    long long s = (cus + wgs - 1) / wgs;
    const long long max_s = (span + 32 * kKeySets - 1) / (32 * kKeySets);
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    splits = (int)s;
  }
  if (splits > 4096) return fail(WPTV_E_INVALID, "verify_attention: splits %d above 4096", splits);
  p.splits = splits;
  if (splits > 1) {
    const size_t rows = (size_t)B * p.groups * splits * 16 * p.mbw;
    p.bytes = align_up(rows * c * sizeof(float), 256) + align_up(rows * sizeof(float), 256);
  } else {
    p.bytes = 0;
  }
  *out = p;
  return WPTV_OK;
}

template <int C, int MBW, bool TREE>
void launch_mfma(dim3 grid, hipStream_t stream, const unsigned short* q, const unsigned short* k, int64_t ksb,
                 int64_t ksn, const unsigned short* v, int64_t vsb, int64_t vsn, const int64_t* positions,
                 int window, const int64_t* tree_base, const uint64_t* ancestors, const float* sink, int T, int H,
                 int N, float scale_log2, int groups, int splits, int range_from_positions, int xcd_map,
                 unsigned short* out, float* lse, float* part_o, float* part_lse) {
  hipLaunchKernelGGL((verify_attention_mfma<C, MBW, TREE>), grid, dim3(kKeySets * MBW * 64), 0, stream, q, k, ksb,
                     ksn, v, vsb, vsn, positions, window, tree_base, ancestors, sink, T, H, N, scale_log2, groups,
                     splits, range_from_positions, xcd_map, out, lse, part_o, part_lse);
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

extern "C" int wptv_verify_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                     const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                     const int64_t* positions, int window, const int64_t* tree_base,
                                     const uint64_t* tree_ancestors, const float* sink, int B, int T, int H, int c,
                                     int N, float scale, int splits, int flags, void* out, float* lse,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!q || !k || !v || !positions || !out)
    return fail(WPTV_E_INVALID, "verify_attention: q, k, v, positions and out must be given");
  if ((tree_base == nullptr) != (tree_ancestors == nullptr))
    return fail(WPTV_E_INVALID, "verify_attention: tree_base and tree_ancestors go together");
  if (k_stride_n < c || v_stride_n < c)
    return fail(WPTV_E_INVALID, "verify_attention: a row stride below the head width");
  Plan p;
  int st = plan(B, T, H, c, N, window, dtype, flags, splits, &p);
  if (st != WPTV_OK) return st;
  const float scale_log2 = scale * kLog2e;
  if (p.mfma) {
    // 32-bit byte offsets within one batch row's table (buffer loads).
    const bool ok_range = (double)N * (double)(k_stride_n > v_stride_n ? k_stride_n : v_stride_n) * 2.0 < 4.0e9;
    const bool ok_align = ok_range && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && (k_stride_b % 8 == 0) &&
                          (k_stride_n % 8 == 0) && (v_stride_b % 8 == 0) && (v_stride_n % 8 == 0);
    if (!ok_align) p.mfma = false, p.splits = 1, p.bytes = 0;
  }
  if (!p.mfma) {
    dim3 grid(T * H, B);
    if (dtype == WPTV_F32)
      hipLaunchKernelGGL(attention_generic<float>, grid, dim3(64), 0, stream, (const float*)q, (const float*)k,
                         k_stride_b, k_stride_n, (const float*)v, v_stride_b, v_stride_n, nullptr, 0, positions,
                         window, tree_base, tree_ancestors, sink, T, H, c, N, scale_log2, (float*)out, lse);
    else
      hipLaunchKernelGGL(attention_generic<unsigned short>, grid, dim3(64), 0, stream, (const unsigned short*)q,
                         (const unsigned short*)k, k_stride_b, k_stride_n, (const unsigned short*)v, v_stride_b,
                         v_stride_n, nullptr, 0, positions, window, tree_base, tree_ancestors, sink, T, H, c, N,
                         scale_log2, (unsigned short*)out, lse);
    return launched("attention_generic");
  }
  if (p.bytes > 0 && (!workspace || workspace_bytes < p.bytes))
    return fail(WPTV_E_INVALID, "verify_attention: workspace of %zu bytes, %zu needed for %d splits",
                workspace_bytes, p.bytes, p.splits);
  const int R = T * H;
  const int rows_per_group = 16 * p.mbw;
  float* part_o = nullptr;
  float* part_lse = nullptr;
  if (p.splits > 1) {
    const size_t rows = (size_t)B * p.groups * p.splits * rows_per_group;
    part_o = static_cast<float*>(workspace);
    part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(rows * c * sizeof(float), 256));
  }
  const int units = B * p.groups;
  dim3 grid(units * p.splits);
  const int xcd_map = units % 8 == 0 ? 1 : 0;
  // Full causal attention of a single query group reads the whole table; any
  // other case takes its key range from the positions.
  const int from_positions = (window > 0 || p.groups > 1 || (flags & WPTV_ATTN_RANGE_FROM_POSITIONS)) ? 1 : 0;
  const auto* qb = static_cast<const unsigned short*>(q);
  const auto* kb = static_cast<const unsigned short*>(k);
  const auto* vb = static_cast<const unsigned short*>(v);
  auto* ob = static_cast<unsigned short*>(out);
#define WPTV_LAUNCH(CC, MM)                                                                                     \
  (tree_base ? launch_mfma<CC, MM, true> : launch_mfma<CC, MM, false>)(                                         \
      grid, stream, qb, kb, k_stride_b, k_stride_n, vb, v_stride_b, v_stride_n, positions, window, tree_base,   \
      tree_ancestors, sink, T, H, N, scale_log2, p.groups, p.splits, from_positions, xcd_map, ob, lse, part_o, \
      part_lse)
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
  st = launched("verify_attention_mfma");
  if (st != WPTV_OK || p.splits == 1) return st;
  const int threads = 256;
  const long long items = (long long)B * R * (c / 4);
  dim3 cgrid((unsigned)((items + threads - 1) / threads));
  hipLaunchKernelGGL(combine_splits<unsigned short>, cgrid, dim3(threads), 0, stream, part_o, part_lse, sink, B, R, H, c,
                     rows_per_group, p.groups, p.splits, ob, lse);
  return launched("combine_splits");
}

extern "C" int wptv_sparse_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                     const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                     const int64_t* idx, int K, const int64_t* positions, int window,
                                     const float* sink, int B, int T, int H, int c, int N, float scale, void* out,
                                     float* lse, hipStream_t stream) {
  if (!q || !k || !v || !positions || !out || (K > 0 && !idx))
    return fail(WPTV_E_INVALID, "sparse_attention: q, k, v, positions, out (and idx when K > 0) must be given");
  if (B <= 0 || T <= 0 || H <= 0 || c <= 0 || N <= 0 || K < 0 || window < 0)
    return fail(WPTV_E_INVALID, "sparse_attention: bad shape B=%d T=%d H=%d c=%d N=%d K=%d window=%d", B, T, H, c,
                N, K, window);
  if (c > kMaxC) return fail(WPTV_E_UNSUPPORTED, "sparse_attention: head width %d above %d", c, kMaxC);
  if (k_stride_n < c || v_stride_n < c)
    return fail(WPTV_E_INVALID, "sparse_attention: a row stride below the head width");
  const float scale_log2 = scale * kLog2e;
  const int64_t* rows = K > 0 ? idx : nullptr;
  dim3 grid(T * H, B);
  if (dtype == WPTV_F32)
    hipLaunchKernelGGL(attention_generic<float>, grid, dim3(64), 0, stream, (const float*)q, (const float*)k, k_stride_b,
                       k_stride_n, (const float*)v, v_stride_b, v_stride_n, rows, K, positions, window, nullptr,
                       nullptr, sink, T, H, c, N, scale_log2, (float*)out, lse);
  else if (dtype == WPTV_BF16)
    hipLaunchKernelGGL(attention_generic<unsigned short>, grid, dim3(64), 0, stream, (const unsigned short*)q,
                       (const unsigned short*)k, k_stride_b, k_stride_n, (const unsigned short*)v, v_stride_b,
                       v_stride_n, rows, K, positions, window, nullptr, nullptr, sink, T, H, c, N, scale_log2,
                       (unsigned short*)out, lse);
  else
    return fail(WPTV_E_UNSUPPORTED, "sparse_attention: dtype %d is neither fp32 nor bf16", dtype);
  return launched("attention_generic");
}
