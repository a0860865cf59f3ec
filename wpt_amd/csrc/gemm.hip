// Skinny matrix products of the verify step on the matrix cores:
//
//   C[M, N] = X[M, K] . W[N, K]^T        bf16 in, FP32 accumulation
//
// The reference's projections and lm_head are nn.Linear products under bf16
// autocast (attention.py:113-124,157-168, layers.py:45-61, model.py:267,471):
// the verify step multiplies M = B (k+1) rows (160 at batch 32, k = 4) by
// weights of 8 to 134 MB, so each product streams its weight matrix once and
// the rows X stay in the L2.
//
// One workgroup (4 wavefronts) per 64 output columns and one part of K (a
// "split"; the splits of a column tile add their FP32 products into the
// workspace, and wptv_gemm's reduction, or the consumer, sums them).  The
// workgroup stages 64-wide K chunks of W (64 rows) and of X (all M rows,
// padded to a multiple of 32) through a ring in LDS by DMA; each wavefront
// multiplies its share of the 16-row blocks of X by the four 16-column blocks
// of W:
//
//   C^T[n, m] += W[n, k] . X^T[k, m]     v_mfma_f32_16x16x32_bf16, W as the A
//                                       operand, so lane (j, g) ends with 4
//                                       consecutive columns of row m = j
//
// LDS rows are 128 bytes (64 bf16); the 16-byte piece q of row r sits at
// position q ^ ((r >> 1) & 7), so the 16 lanes of an operand read (16 rows,
// one piece) hit distinct bank groups.  The DMA writes 1 KiB (8 rows) per
// instruction, each lane fetching the piece that belongs at its position.
#include "wptv_common.h"

#include <climits>

namespace wptv {
namespace {

constexpr int kGemmWaves = 4;
constexpr int kTileN = 64;         // output columns per workgroup (the wide form: 128)
constexpr int kChunkK = 64;        // K per staged chunk (two k-steps of 32)
constexpr int kRowBytes = kChunkK * 2;

// R32: the staged X rows, 32 R32 (all M rows, padded to a multiple of 32);
// TN: the workgroup's output columns (64, or 128 where the column tiles
// outnumber the compute units: half the X re-reads per weight byte).
template <int R32, int TN = kTileN>
struct GemmTile {
  static constexpr int kRows = 32 * R32;
  static constexpr int kBlocks = kRows / 16;                        // 16-row blocks
  static constexpr int kMaxPerWave = (kBlocks + kGemmWaves - 1) / kGemmWaves;
  static constexpr int kNBlocks = TN / 16;                          // 16-column blocks
  static constexpr int kWPieces = TN / 8;                           // 1 KiB W pieces (8 rows) per chunk
  static constexpr int kWBytes = TN * kRowBytes;                    // 8 or 16 KiB
  static constexpr int kSlotBytes = kWBytes + kRows * kRowBytes;
  static constexpr int kSlots = (160 * 1024) / kSlotBytes < 4 ? (160 * 1024) / kSlotBytes : 4;
  static constexpr int kPieces = kSlotBytes / 1024;                 // 1 KiB DMA instructions per chunk
  static constexpr int kPerWave = kPieces / kGemmWaves;             // TN / 32 + R32
  static_assert(kPieces % kGemmWaves == 0, "pieces per wave");
  static_assert(kSlots >= 2, "ring");
  static_assert((kSlots - 1) * kPerWave < 64, "vmcnt range");
};

__device__ __forceinline__ int gemm_swz(int r) { return (r >> 1) & 7; }

// vmcnt wait for this wavefront's pieces of one chunk, `behind` chunks
// (0 .. kSlots - 1) still allowed in flight after it.
template <int kPer>
__device__ __forceinline__ void wait_chunks_behind(int behind) {
  if (behind >= 3)
    wait_vmcnt<(3 * kPer < 64 ? 3 * kPer : 63)>();
  else if (behind == 2)
    wait_vmcnt<2 * kPer>();
  else if (behind == 1)
    wait_vmcnt<kPer>();
  else
    wait_vmcnt<0>();
}

enum GemmOut { kPartF32 = 0, kOutBf16 = 1, kOutF32 = 2, kOutSwiGLU = 3 };

// silu(g) * u of the bf16-rounded halves, rounded once to bf16: what the
// product rounded to bf16 and then wptv_swiglu give.
__device__ __forceinline__ unsigned short swiglu_bf16(float g, float u) {
  const float gb = bf16_to_f32(f32_to_bf16(g)), ub = bf16_to_f32(f32_to_bf16(u));
  return f32_to_bf16(gb / (1.f + expf(-gb)) * ub);
}

// grid: (N / 64, splits).  Split z multiplies K chunks [z cps, min((z + 1) cps, K / 64)).
// OUT: kPartF32 -> part[z][m][n] FP32; kOutBf16 -> out bf16; kOutF32 -> out
// FP32 holding the bf16-rounded product (the reference's bf16 product cast to
// FP32); kOutSwiGLU -> out bf16 [M, N / 2] = silu(gate) * up, the weight's 64
// rows of a column tile being 32 gate rows then the 32 up rows of the same
// features (wptv_gemm_swiglu).
template <int R32, int OUT, int TN = kTileN>
__global__ __launch_bounds__(kGemmWaves * 64, 1) void gemm_xwt(const unsigned short* __restrict__ x, int64_t ldx,
                                                               const unsigned short* __restrict__ w, int64_t ldw,
                                                               int M, int N, int K, int cps, void* __restrict__ out,
                                                               int64_t ldo) {
  using G = GemmTile<R32, TN>;
  constexpr int MBW = G::kMaxPerWave;
  constexpr int NB = G::kNBlocks;
  static_assert(OUT != kOutSwiGLU || TN == kTileN, "the SwiGLU epilogue pairs 32 gate and 32 up columns of a 64-column tile");
  __shared__ __attribute__((aligned(16))) unsigned char ring[G::kSlots * G::kSlotBytes];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * TN;
  const int z = blockIdx.y;
  const int chunks = K / kChunkK;
  const int c0 = z * cps;
  const int nch = max(0, min(chunks, c0 + cps) - c0);

  // DMA: piece p of a chunk is 8 rows x 128 bytes (W rows for p < TN / 8, then X
  // rows); lane l fills row rr = l / 8, position pos = l % 8.  The row part of
  // the offset and the chunk's K offset go in the scalar offset.
  const i32x4 wrs = buffer_resource(w);
  const i32x4 xrs = buffer_resource(x);
  const int rr = lane >> 3, pos = lane & 7;
  const uint32_t ldw_b = (uint32_t)ldw * 2u, ldx_b = (uint32_t)ldx * 2u;
  // the swizzle of row 8 p' + rr depends on p' only through p' & 1
  const uint32_t wv_off[2] = {(uint32_t)rr * ldw_b + 16u * (uint32_t)(pos ^ gemm_swz(rr)),
                              (uint32_t)rr * ldw_b + 16u * (uint32_t)(pos ^ gemm_swz(8 + rr))};
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  auto issue = [&](int i) {  // this wavefront's pieces of chunk c0 + i
    const uint32_t slot = ring_lds + (uint32_t)(i % G::kSlots) * G::kSlotBytes;
    const uint32_t kb = (uint32_t)(c0 + i) * kRowBytes;
#pragma unroll
    for (int u = 0; u < G::kPerWave; ++u) {
      const int p = wv + kGemmWaves * u;
      if (p < G::kWPieces) {
        const uint32_t sbase = (uint32_t)(n0 + 8 * p) * ldw_b + kb;
        dma_16B_at(wrs, wv_off[p & 1], sbase, slot + 1024u * p);
      } else {
        const int row = 8 * (p - G::kWPieces) + rr;
        const int src = row < M ? row : M - 1;  // padding rows repeat row M - 1
        dma_16B(xrs, (uint32_t)src * ldx_b + kb + 16u * (uint32_t)(pos ^ gemm_swz(row)), slot + 1024u * p);
      }
    }
  };
#pragma unroll
  for (int i = 0; i < G::kSlots - 1; ++i)
    if (i < nch) issue(i);

  // operand offsets within a slot: W row 16 nb + j and X row 16 mb + j,
  // piece 4 s + g (s = k-step within the chunk)
  uint32_t op_off[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) op_off[s] = (uint32_t)(j * kRowBytes + 16 * ((4 * s + g) ^ gemm_swz(j)));
  // this wavefront's 16-row blocks: mb0 .. mb0 + nblk - 1 (the blocks are
  // dealt out as evenly as they go)
  constexpr int kBase = G::kBlocks / kGemmWaves, kExtra = G::kBlocks % kGemmWaves;
  const int nblk = kBase + (wv < kExtra ? 1 : 0);
  const int mb0 = wv * kBase + min(wv, kExtra);
  f32x4 acc[MBW][NB];
#pragma unroll
  for (int i = 0; i < MBW; ++i)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[i][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
  for (int i = 0; i < nch; ++i) {
    // chunk i has landed (this wavefront's pieces; the barrier covers the others')
    wait_chunks_behind<G::kPerWave>(min(nch - 1 - i, G::kSlots - 2));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // the slot of chunk i - 1 is free (every wavefront is past it): refill it
    if (i + G::kSlots - 1 < nch) issue(i + G::kSlots - 1);
    const unsigned char* st = ring + (i % G::kSlots) * G::kSlotBytes;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 wf[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        wf[nb] = *reinterpret_cast<const bf16x8*>(st + 16 * nb * kRowBytes + op_off[s]);
#pragma unroll
      for (int ii = 0; ii < MBW; ++ii) {
        if (ii >= nblk || 16 * (mb0 + ii) >= M) break;  // not this wavefront's, or padding rows only
        const bf16x8 xf = *reinterpret_cast<const bf16x8*>(st + G::kWBytes + 16 * (mb0 + ii) * kRowBytes + op_off[s]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[ii][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[nb], xf, acc[ii][nb], 0, 0, 0);
      }
    }
  }
  wait_vmcnt<0>();

  // lane (j, g) holds columns n0 + 16 nb + 4 g .. + 3 of row 16 mb + j
#pragma unroll
  for (int ii = 0; ii < MBW; ++ii) {
    const int m = 16 * (mb0 + ii) + j;
    if (ii >= nblk || m >= M) continue;
    if constexpr (OUT == kOutSwiGLU) {
      // blocks 0, 1: gate of features n0 / 2 + 16 nb + 4 g .. + 3; blocks 2, 3: their up
      typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const f32x4 gv = acc[ii][nb], uv = acc[ii][nb + 2];
        unsigned short* dst = static_cast<unsigned short*>(out) + (int64_t)m * ldo + n0 / 2 + 16 * nb + 4 * g;
        *reinterpret_cast<u16x4*>(dst) = u16x4{swiglu_bf16(gv[0], uv[0]), swiglu_bf16(gv[1], uv[1]),
                                               swiglu_bf16(gv[2], uv[2]), swiglu_bf16(gv[3], uv[3])};
      }
      continue;
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = n0 + 16 * nb + 4 * g;
      const f32x4 a = acc[ii][nb];
      // parts and bf16 outputs (the lm_head's logits) are read once, by another kernel: written non-temporally
      if constexpr (OUT == kPartF32) {
        float* dst = static_cast<float*>(out) + ((int64_t)z * M + m) * N + n;
        __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(dst));
      } else if constexpr (OUT == kOutBf16) {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        unsigned short* dst = static_cast<unsigned short*>(out) + (int64_t)m * ldo + n;
        const bf16x4 r = bf16x4{static_cast<__bf16>(a[0]), static_cast<__bf16>(a[1]), static_cast<__bf16>(a[2]),
                                static_cast<__bf16>(a[3])};
        __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, r), reinterpret_cast<uint64_t*>(dst));
      } else {
        float* dst = static_cast<float*>(out) + (int64_t)m * ldo + n;
        *reinterpret_cast<f32x4*>(dst) =
            f32x4{bf16_to_f32(f32_to_bf16(a[0])), bf16_to_f32(f32_to_bf16(a[1])), bf16_to_f32(f32_to_bf16(a[2])),
                  bf16_to_f32(f32_to_bf16(a[3]))};
      }
    }
  }
}

// out[m, n] = sum over the splits of part[z][m][n], as bf16, or as FP32
// holding the bf16-rounded sum.  One thread per 4 columns.
template <bool F32>
__global__ __launch_bounds__(256) void gemm_reduce(const float* __restrict__ part, int splits, int M, int N,
                                                   void* __restrict__ out, int64_t ldo) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = N / 4;
  if (idx >= (int64_t)M * per_row) return;
  const int m = (int)(idx / per_row), n = (int)(idx % per_row) * 4;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int z = 0; z < splits; ++z) s += *reinterpret_cast<const f32x4*>(part + ((int64_t)z * M + m) * N + n);
  if constexpr (F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + (int64_t)m * ldo + n) =
        f32x4{bf16_to_f32(f32_to_bf16(s[0])), bf16_to_f32(f32_to_bf16(s[1])), bf16_to_f32(f32_to_bf16(s[2])),
              bf16_to_f32(f32_to_bf16(s[3]))};
  } else {
    typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<u16x4*>(static_cast<unsigned short*>(out) + (int64_t)m * ldo + n) =
        u16x4{f32_to_bf16(s[0]), f32_to_bf16(s[1]), f32_to_bf16(s[2]), f32_to_bf16(s[3])};
  }
}

constexpr int kMaxGemmRows = 512;  // 8 row blocks per wavefront
// Above this many rows an unsplit product runs on the wide tiles (gemm_wide.hip):
// measured on the MI355X at the lm_head's 32768 x 2048, the skinny product
// reaches hipBLASLt's time up to 320 rows only.
constexpr int kWideMinRows = 321;

struct GemmPlan {
  int r32;     // staged X rows / 32
  int splits;  // parts of K
  int cps;     // K chunks per split
  int tn;      // output columns per workgroup
  size_t bytes;
  bool wide;   // the 256 x 256 tiles of gemm_wide
};

int gemm_plan(int M, int N, int K, int requested, GemmPlan* p, bool allow_wide = false) {
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(WPTV_E_INVALID, "gemm: M, N and K must be positive (got %d, %d, %d)", M, N, K);
  p->wide = false;
  if (allow_wide && M >= kWideMinRows && requested <= 0 && gemm_wide_fits(M, N, K)) {
    p->wide = true;
    p->r32 = 0;
    p->splits = 1;
    p->cps = K / kChunkK;
    p->tn = 256;
    p->bytes = 0;
    return WPTV_OK;
  }
  if (M > kMaxGemmRows) return fail(WPTV_E_UNSUPPORTED, "gemm: M = %d above %d rows", M, kMaxGemmRows);
  if (N % kTileN || K % kChunkK)
    return fail(WPTV_E_UNSUPPORTED, "gemm: N (%d) must be a multiple of %d and K (%d) of %d", N, kTileN, K, kChunkK);
  // instantiated row counts: 32 r32 for r32 in 1-6, 8, 10, 12, 16
  int r32 = (M + 31) / 32;
  if (r32 > 6) r32 = r32 <= 8 ? 8 : r32 <= 10 ? 10 : r32 <= 12 ? 12 : 16;
  const int tiles = N / kTileN, chunks = K / kChunkK;
  int s = requested;
  if (s <= 0) {
    s = compute_units() / tiles;  // one workgroup per compute unit
    if (s < 1) s = 1;
  }
  if (s > chunks) s = chunks;
  const int cps = (chunks + s - 1) / s;
  s = (chunks + cps - 1) / cps;  // no empty split
  p->r32 = r32;
  p->splits = s;
  p->cps = cps;
  // one part and at least two 64-column tiles per compute unit (an lm_head):
  // 128-column tiles, each reading X once for twice the weights
  p->tn = (s == 1 && N % (2 * kTileN) == 0 && tiles >= 2 * compute_units()) ? 2 * kTileN : kTileN;
  p->bytes = s > 1 ? align_up((size_t)s * M * N * sizeof(float), 256) : 0;
  return WPTV_OK;
}

template <int R32, int OUT, int TN>
void launch_gemm(dim3 grid, hipStream_t stream, const unsigned short* x, int64_t ldx, const unsigned short* w,
                 int64_t ldw, int M, int N, int K, int cps, void* out, int64_t ldo) {
  hipLaunchKernelGGL((gemm_xwt<R32, OUT, TN>), grid, dim3(kGemmWaves * 64), 0, stream, x, ldx, w, ldw, M, N, K, cps,
                     out, ldo);
}

template <int OUT, int TN = kTileN>
void launch_gemm_rows(int r32, dim3 grid, hipStream_t stream, const unsigned short* x, int64_t ldx,
                      const unsigned short* w, int64_t ldw, int M, int N, int K, int cps, void* out, int64_t ldo) {
#define WPTV_G(RR) launch_gemm<RR, OUT, TN>(grid, stream, x, ldx, w, ldw, M, N, K, cps, out, ldo)
  switch (r32) {
    case 1: WPTV_G(1); break;
    case 2: WPTV_G(2); break;
    case 3: WPTV_G(3); break;
    case 4: WPTV_G(4); break;
    case 5: WPTV_G(5); break;
    case 6: WPTV_G(6); break;
    case 8: WPTV_G(8); break;
    case 10: WPTV_G(10); break;
    case 12: WPTV_G(12); break;
    default: WPTV_G(16); break;
  }
#undef WPTV_G
}

}  // namespace
}  // namespace wptv

using namespace wptv;

extern "C" int wptv_gemm_workspace(int M, int N, int K, int* splits, size_t* bytes) {
  if (!splits || !bytes) return fail(WPTV_E_INVALID, "gemm_workspace: null output pointer");
  GemmPlan p;
  const int st = gemm_plan(M, N, K, *splits, &p, true);
  if (st != WPTV_OK) return st;
  *splits = p.splits;
  *bytes = p.bytes;
  return WPTV_OK;
}

extern "C" int wptv_gemm_parts(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K,
                               int splits, float* parts, size_t parts_bytes, hipStream_t stream) {
  if (!x || !w || !parts) return fail(WPTV_E_INVALID, "gemm_parts: x, w and parts must be given");
  GemmPlan p;
  const int st = gemm_plan(M, N, K, splits, &p);
  if (st != WPTV_OK) return st;
  if (p.splits != splits) return fail(WPTV_E_INVALID, "gemm_parts: %d splits do not cut K = %d evenly into chunks "
                                                      "(%d would); take the count from wptv_gemm_workspace",
                                      splits, K, p.splits);
  if (ldx < K || ldw < K) return fail(WPTV_E_INVALID, "gemm_parts: a leading dimension below the row width");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(parts, 16) || ldx % 8 || ldw % 8)
    return fail(WPTV_E_INVALID, "gemm_parts: x, w and parts must be 16-byte aligned with leading dimensions of 8");
  if ((double)N * (double)ldw * 2.0 >= 4.0e9 || (double)M * (double)ldx * 2.0 >= 4.0e9)
    return fail(WPTV_E_UNSUPPORTED, "gemm_parts: operands above 4 GB");
  const size_t need = (size_t)p.splits * M * N * sizeof(float);
  if (parts_bytes < need)
    return fail(WPTV_E_INVALID, "gemm_parts: %zu bytes of parts, %zu needed", parts_bytes, need);
  dim3 grid(N / kTileN, p.splits);
  launch_gemm_rows<kPartF32>(p.r32, grid, stream, static_cast<const unsigned short*>(x), ldx,
                            static_cast<const unsigned short*>(w), ldw, M, N, K, p.cps, parts, 0);
  return launched("gemm_xwt");
}

extern "C" int wptv_gemm_swiglu(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out,
                                int64_t ldo, hipStream_t stream) {
  if (!x || !w || !out) return fail(WPTV_E_INVALID, "gemm_swiglu: x, w and out must be given");
  GemmPlan p;
  const int st = gemm_plan(M, N, K, 1, &p);  // one part: the epilogue needs the whole sum
  if (st != WPTV_OK) return st;
  if (ldx < K || ldw < K || ldo < N / 2)
    return fail(WPTV_E_INVALID, "gemm_swiglu: a leading dimension below the row width");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 8) || ldx % 8 || ldw % 8 || ldo % 4)
    return fail(WPTV_E_INVALID, "gemm_swiglu: x and w 16-byte aligned, leading dimensions of 8 (out: 4) elements");
  if ((double)N * (double)ldw * 2.0 >= 4.0e9 || (double)M * (double)ldx * 2.0 >= 4.0e9)
    return fail(WPTV_E_UNSUPPORTED, "gemm_swiglu: operands above 4 GB");
  dim3 grid(N / kTileN, 1);
  launch_gemm_rows<kOutSwiGLU>(p.r32, grid, stream, static_cast<const unsigned short*>(x), ldx,
                               static_cast<const unsigned short*>(w), ldw, M, N, K, p.cps, out, ldo);
  return launched("gemm_xwt");
}

extern "C" int wptv_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out,
                         int64_t ldo, int out_dtype, int splits, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (!x || !w || !out) return fail(WPTV_E_INVALID, "gemm: x, w and out must be given");
  if (out_dtype != WPTV_BF16 && out_dtype != WPTV_F32)
    return fail(WPTV_E_UNSUPPORTED, "gemm: output dtype %d is neither bf16 nor fp32", out_dtype);
  GemmPlan p;
  int st = gemm_plan(M, N, K, splits, &p, true);
  if (st != WPTV_OK) return st;
  if (ldx < K || ldw < K || ldo < N) return fail(WPTV_E_INVALID, "gemm: a leading dimension below the row width");
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(out, 16) || ldx % 8 || ldw % 8 || ldo % 4)
    return fail(WPTV_E_INVALID, "gemm: x, w and out must be 16-byte aligned with leading dimensions of 8 elements");
  if ((double)N * (double)ldw * 2.0 >= 4.0e9 || (double)M * (double)ldx * 2.0 >= 4.0e9)
    return fail(WPTV_E_UNSUPPORTED, "gemm: operands above 4 GB");
  if (p.splits > 1 && (!workspace || workspace_bytes < p.bytes))
    return fail(WPTV_E_INVALID, "gemm: workspace of %zu bytes, %zu needed for %d splits", workspace_bytes, p.bytes,
                p.splits);
  if (p.wide) return gemm_wide(x, ldx, w, ldw, M, N, K, out, ldo, out_dtype, stream);
  const auto* xb = static_cast<const unsigned short*>(x);
  const auto* wb = static_cast<const unsigned short*>(w);
  dim3 grid(N / p.tn, p.splits);
  if (p.splits == 1) {
    if (p.tn != kTileN) {
      if (out_dtype == WPTV_BF16)
        launch_gemm_rows<kOutBf16, 2 * kTileN>(p.r32, grid, stream, xb, ldx, wb, ldw, M, N, K, p.cps, out, ldo);
      else
        launch_gemm_rows<kOutF32, 2 * kTileN>(p.r32, grid, stream, xb, ldx, wb, ldw, M, N, K, p.cps, out, ldo);
    } else if (out_dtype == WPTV_BF16) {
      launch_gemm_rows<kOutBf16>(p.r32, grid, stream, xb, ldx, wb, ldw, M, N, K, p.cps, out, ldo);
    } else {
      launch_gemm_rows<kOutF32>(p.r32, grid, stream, xb, ldx, wb, ldw, M, N, K, p.cps, out, ldo);
    }
    return launched("gemm_xwt");
  }
  launch_gemm_rows<kPartF32>(p.r32, grid, stream, xb, ldx, wb, ldw, M, N, K, p.cps, workspace, 0);
  st = launched("gemm_xwt");
  if (st != WPTV_OK) return st;
  const long long items = (long long)M * (N / 4);
  dim3 rgrid((unsigned)((items + 255) / 256));
  if (out_dtype == WPTV_BF16)
    hipLaunchKernelGGL(gemm_reduce<false>, rgrid, dim3(256), 0, stream, static_cast<const float*>(workspace), p.splits,
                       M, N, out, ldo);
  else
    hipLaunchKernelGGL(gemm_reduce<true>, rgrid, dim3(256), 0, stream, static_cast<const float*>(workspace), p.splits,
                       M, N, out, ldo);
  return launched("gemm_reduce");
}
