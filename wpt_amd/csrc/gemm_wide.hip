// Matrix products over many rows on the matrix cores:
//
//   C[M, N] = X[M, K] . W[N, K]^T        bf16 in, FP32 accumulation
//
// the reference's lm_head under bf16 autocast (model.py:471: head(final_norm(h)))
// when a reading holds more rows than the skinny products serve well: the tree
// verification scores 16 batch rows x 31 draft nodes = 496 rows against the
// [32768 x 2048] head, 66.6 GFLOP over 134 MB of weights (331 flop per byte,
// at the bf16 ridge of the MI355X), so the product has to keep the matrix
// cores busy rather than stream its weights.
//
// One workgroup of eight wavefronts (two per SIMD) per 256 x 256 output tile;
// at 496 rows and 32768 columns that is 2 x 128 = 256 workgroups, one per
// compute unit.  The workgroup stages 32-wide K chunks of both operands
// (256 rows x 64 bytes each, 32 KiB a chunk) through a four-chunk LDS ring by
// DMA (buffer_load ... lds), three chunks in flight ahead of the one being
// multiplied, one barrier a chunk.  Each wavefront owns 64 output columns x
// 128 rows and multiplies, per 16-wide k-slice,
//
//   C^T[n, m] += W[n, k] . X^T[k, m]     v_mfma_f32_32x32x16_bf16, W as the A
//                                       operand: lane l ends with columns
//                                       8 (i / 4) + 4 (l / 32) + i % 4 of
//                                       row l % 32 in its register i
//
// two 32-column blocks by four 32-row blocks (8 products, 128 accumulator
// registers), reading the next k-slice's six operand fragments from LDS while
// the current slice's products run; the two wavefronts of a SIMD fill each
// other's LDS waits.  LDS rows are 64 bytes; the 16-byte piece p of row r sits
// at position p ^ ((r >> 1 ^ r >> 2) & 3), so that any 8 (or 16) consecutive
// rows read at one piece cover distinct banks.
//
// The tile's 256 x 256 results leave through LDS: rounded to bf16 (the
// autocast product's dtype), written into the drained ring as [m][n] rows of
// 512 bytes (16-byte piece q of row m at q ^ (m & 7)), then stored 16 bytes a
// lane along whole output rows, as bf16 or as the bf16 values widened to FP32
// (the reference's .float() of the bf16 logits).
//
// Workgroups are dealt to the 8 XCDs in turn; the row tiles of one column tile
// take consecutive slots of one XCD, so its weights come from HBM once and
// from that XCD's L2 for the other row tiles.
#include "wptv_common.h"

#include <climits>

namespace wptv {
namespace {

constexpr int kWideWaves = 8;
constexpr int kWideTile = 256;               // output rows and columns of a workgroup
constexpr int kWideChunk = 32;               // K per staged chunk
constexpr int kWideRow = kWideChunk * 2;     // bytes of one staged row
constexpr int kWideHalf = kWideTile * kWideRow;  // 16 KiB: one operand's chunk
constexpr int kWideStage = 2 * kWideHalf;        // 32 KiB: X then W
constexpr int kWideStages = 4;
constexpr int kWidePerWave = kWideStage / 1024 / kWideWaves;  // 1 KiB DMA pieces a wavefront issues per chunk
constexpr int kWideSlices = kWideChunk / 16;                  // k-slices of the 32x32x16 products per chunk
constexpr float kNegInfW = -__builtin_inff();
static_assert(kWideStages * kWideStage >= kWideTile * kWideTile * 2, "the output tile is staged in the ring");
static_assert(kWidePerWave == 4, "two X and two W pieces a wavefront");

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int wide_swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// vmcnt wait for this wavefront's pieces of a chunk with `later` of its
// later chunks (0 .. 2) still allowed in flight.
__device__ __forceinline__ void wide_wait(int later) {
  if (later >= 2)
    wait_vmcnt<2 * kWidePerWave>();
  else if (later == 1)
    wait_vmcnt<kWidePerWave>();
  else
    wait_vmcnt<0>();
}

// s_waitcnt lgkmcnt(0), the other counters left alone (gfx9 encoding).
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
  asm volatile("" ::: "memory");
}

// grid: row_tiles x (N / 256) workgroups, 512 threads.  OUT: kWideBf16 or
// kWideF32.  FM false: x and w row-major with leading dimensions ldx, ldw;
// FM true: both in the fm layout (wptv_common.h), x with ldx row blocks (at
// least 2 ceil(M / 32)), w with ldw = N / 16.
// kWideArgmax: no product stored; each row's largest bf16-rounded value over
// the tile's 256 columns and its first index, as a (value, index) pair at
// out[column tile * M + row] (the greedy decisions' first maximal index,
// reduced over the column tiles by wide_argmax_reduce).
enum WideOut { kWideBf16 = 0, kWideF32 = 1, kWideArgmax = 2 };

// torch.argmax's order: a NaN above every number, then the larger value;
// the lower index among equals (NaNs included).
__device__ __forceinline__ void wide_better(float& v, int& i, float v2, int i2) {
  const bool nan = v != v, nan2 = v2 != v2;
  if (nan2 ? (!nan || i2 < i) : (!nan && (v2 > v || (v2 == v && i2 < i)))) {
    v = v2;
    i = i2;
  }
}

template <int OUT, bool FM>
__global__ __launch_bounds__(kWideWaves * 64, 1) void gemm_wide(const unsigned short* __restrict__ x, int64_t ldx,
                                                                const unsigned short* __restrict__ w, int64_t ldw,
                                                                int M, int N, int K, int row_tiles,
                                                                void* __restrict__ out, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) unsigned char ring[kWideStages * kWideStage];  // 128 KiB

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col_tiles = N / kWideTile;
  int rt, ct;
  {
    const int id = blockIdx.x;
    if (col_tiles % 8 == 0) {  // slot s of XCD x: column tile 8 (s / row_tiles) + x, row tile s % row_tiles
      const int xcd = id & 7, slot = id >> 3;
      rt = slot % row_tiles;
      ct = (slot / row_tiles) * 8 + xcd;
    } else {
      rt = id % row_tiles;
      ct = id / row_tiles;
    }
  }
  const int m0 = rt * kWideTile, n0 = ct * kWideTile;
  const int chunks = K / kWideChunk;

  // DMA: a chunk is 32 pieces of 1 KiB (16 rows x 64 bytes): X rows in pieces
  // 0-15, W rows in 16-31; wavefront wv issues X and W pieces 2 wv and 2 wv + 1.
  // Row-major operands: lane l fills row rr = l / 4 of a piece at position
  // pos = l % 4, fetching the row's global piece pos ^ swz(row).  fm operands:
  // a piece is one fm block (16 rows of the chunk's 32 columns), 1 KiB
  // contiguous, copied as it lies.  X rows past M repeat row M - 1 (fm: row
  // blocks past the operand's repeat its last block); their products are
  // never stored.
  const i32x4 xrs = buffer_resource(x), wrs = buffer_resource(w);
  uint32_t xoff[2], woff[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if constexpr (FM) {
      const int xb = min(m0 / 16 + 2 * wv + u, (int)ldx - 1);
      xoff[u] = (uint32_t)xb * 1024u + 16u * (uint32_t)lane;
      woff[u] = (uint32_t)(n0 / 16 + 2 * wv + u) * 1024u + 16u * (uint32_t)lane;
    } else {
      const int rr = lane >> 2, pos = lane & 3;
      const int r = 16 * (2 * wv + u) + rr;
      const int xm = min(m0 + r, M - 1);
      xoff[u] = (uint32_t)xm * (uint32_t)ldx * 2u + 16u * (uint32_t)(pos ^ wide_swz(r));
      woff[u] = (uint32_t)(n0 + r) * (uint32_t)ldw * 2u + 16u * (uint32_t)(pos ^ wide_swz(r));
    }
  }
  // the chunk's offset: row-major 64 bytes of every row; fm one k-step of blocks
  const uint32_t xstep = FM ? (uint32_t)ldx * 1024u : (uint32_t)kWideRow;
  const uint32_t wstep = FM ? (uint32_t)ldw * 1024u : (uint32_t)kWideRow;
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_address(ring));
  auto issue = [&](int c) {
    if (c >= chunks) return;
    const uint32_t st = ring_lds + (uint32_t)(c % kWideStages) * kWideStage;
#pragma unroll
    for (int u = 0; u < 2; ++u) dma_16B_at(xrs, xoff[u], (uint32_t)c * xstep, st + 1024u * (2 * wv + u));
#pragma unroll
    for (int u = 0; u < 2; ++u) dma_16B_at(wrs, woff[u], (uint32_t)c * wstep, st + kWideHalf + 1024u * (2 * wv + u));
  };
  // waits until chunk c has landed (its later chunks in flight)
  auto landed = [&](int c) { wide_wait(min(2, max(0, chunks - 1 - c))); };

  // operand fragments: lane l reads row l % 32 of a 32-row block, k-elements
  // 8 (l / 32) .. + 7 of k-slice kk (piece 2 kk + l / 32); a 32-row block is
  // 2 KiB of the stage either way (two fm blocks, in which row j's piece p
  // sits at 256 p + 16 j: any 16 lanes read 256 contiguous bytes)
  const int rl = lane & 31, hl = lane >> 5;
  uint32_t koff[kWideSlices];
#pragma unroll
  for (int kk = 0; kk < kWideSlices; ++kk)
    koff[kk] = FM ? (uint32_t)((rl >> 4) * 1024 + (2 * kk + hl) * 256 + (rl & 15) * 16)
                  : (uint32_t)(rl * kWideRow + 16 * ((2 * kk + hl) ^ wide_swz(rl)));
  const int wn = wv & 3, wm = wv >> 2;  // columns 64 wn .. + 63, rows 128 wm .. + 127 of the tile
  const uint32_t wbase = kWideHalf + (uint32_t)(64 * wn) * kWideRow;
  const uint32_t xbase = (uint32_t)(128 * wm) * kWideRow;

  f32x16 acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;
  bf16x8 wf[kWideSlices][2], xf[kWideSlices][4];

  // Ping-pong: the workgroup runs 2 chunks + 1 phases, a barrier before each.
  // Wavefront group g = wm (one wavefront of each group per SIMD) takes chunk
  // s's operands from LDS into registers in phase 2 s + g and multiplies them
  // in phase 2 s + g + 1, so in every phase one wavefront of a SIMD reads LDS
  // (and issues its DMA pieces for chunk s + 3) while the other runs its 16
  // products.  Chunk s is read in phases 2 s and 2 s + 1 and has landed at
  // the barrier before phase 2 s; its slot is refilled (chunk s + 4) from
  // phase 2 s + 2 on, after both groups have read it.
  auto load = [&](int c) {
    issue(c + 3);
    const unsigned char* st = ring + (c % kWideStages) * kWideStage;
#pragma unroll
    for (int kk = 0; kk < kWideSlices; ++kk) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        wf[kk][j] = *reinterpret_cast<const bf16x8*>(st + wbase + (uint32_t)(32 * j) * kWideRow + koff[kk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xf[kk][i] = *reinterpret_cast<const bf16x8*>(st + xbase + (uint32_t)(32 * i) * kWideRow + koff[kk]);
    }
    wait_lgkm0();  // the slot may be refilled once both groups have passed the next barriers
  };
  auto multiply = [&]() {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kk = 0; kk < kWideSlices; ++kk)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[kk][j], xf[kk][i], acc[j][i], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  issue(0);
  issue(1);
  issue(2);
  if (wm == 0) {
#pragma unroll 1
    for (int s = 0; s < chunks; ++s) {
      landed(s);
      barrier();  // phase 2 s
      load(s);
      barrier();  // phase 2 s + 1
      multiply();
    }
    wait_vmcnt<0>();
    barrier();  // phase 2 chunks
  } else {
    landed(0);
    barrier();  // phase 0
#pragma unroll 1
    for (int s = 0; s < chunks; ++s) {
      barrier();  // phase 2 s + 1
      load(s);
      landed(s + 1);
      barrier();  // phase 2 s + 2
      multiply();
    }
  }

  if constexpr (OUT == kWideArgmax) {
    // lane l holds, of row 128 wm + 32 i + l % 32, the columns 64 wn + 32 j +
    // 8 g + 4 (l / 32) + e of the tile: its first maximum in column order,
    // then the other half-wave's (lane l ^ 32), then the four wavefronts of
    // the row's half through LDS, in column order
    __syncthreads();  // the ring is free
    float* rv = reinterpret_cast<float*>(ring);                // [wm][wn][128]
    int* ri = reinterpret_cast<int*>(ring + 2 * 4 * 128 * 4);  // the same layout
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float bv = kNegInfW;
      int bi = INT_MAX;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          wide_better(bv, bi, bf16_to_f32(f32_to_bf16(acc[j][i][e])),
                      n0 + 64 * wn + 32 * j + 8 * (e >> 2) + 4 * hl + (e & 3));
      const float ov = __shfl_xor(bv, 32, 64);
      const int oi = __shfl_xor(bi, 32, 64);
      wide_better(bv, bi, ov, oi);
      if (hl == 0) {
        rv[(wm * 4 + wn) * 128 + 32 * i + rl] = bv;
        ri[(wm * 4 + wn) * 128 + 32 * i + rl] = bi;
      }
    }
    __syncthreads();
    if (threadIdx.x < kWideTile) {
      const int ml = threadIdx.x, half = ml >> 7, r = ml & 127;
      float bv = kNegInfW;
      int bi = INT_MAX;
#pragma unroll
      for (int u = 0; u < 4; ++u) wide_better(bv, bi, rv[(half * 4 + u) * 128 + r], ri[(half * 4 + u) * 128 + r]);
      if (m0 + ml < M) {
        float2* part = static_cast<float2*>(out) + (int64_t)ct * M + m0 + ml;
        *part = float2{bv, __int_as_float(bi)};
      }
    }
    return;
  }

  // every wavefront is done with the ring: stage the tile as bf16 [m][n]
  __syncthreads();
  typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ml = 128 * wm + 32 * i + rl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int q = 8 * wn + 4 * j + g;  // 16-byte piece of row ml: columns 8 q .. 8 q + 7
        const u16x4 v = {f32_to_bf16(acc[j][i][4 * g]), f32_to_bf16(acc[j][i][4 * g + 1]),
                         f32_to_bf16(acc[j][i][4 * g + 2]), f32_to_bf16(acc[j][i][4 * g + 3])};
        *reinterpret_cast<u16x4*>(ring + ml * 512 + 16 * (q ^ (ml & 7)) + 8 * hl) = v;
      }
    }
  __syncthreads();
  const int q = threadIdx.x & 31;
#pragma unroll 4
  for (int pass = 0; pass < kWideTile / 16; ++pass) {
    const int ml = 16 * pass + (threadIdx.x >> 5);
    const int m = m0 + ml;
    if (m >= M) break;
    const u16x8 v = *reinterpret_cast<const u16x8*>(ring + ml * 512 + 16 * (q ^ (ml & 7)));
    if constexpr (OUT == kWideBf16) {
      *reinterpret_cast<u16x8*>(static_cast<unsigned short*>(out) + (int64_t)m * ldo + n0 + 8 * q) = v;
    } else {
      float* dst = static_cast<float*>(out) + (int64_t)m * ldo + n0 + 8 * q;
      *reinterpret_cast<f32x4*>(dst) = f32x4{bf16_to_f32(v[0]), bf16_to_f32(v[1]), bf16_to_f32(v[2]), bf16_to_f32(v[3])};
      *reinterpret_cast<f32x4*>(dst + 4) =
          f32x4{bf16_to_f32(v[4]), bf16_to_f32(v[5]), bf16_to_f32(v[6]), bf16_to_f32(v[7])};
    }
  }
}

// Each row's first maximal index over the column tiles' (value, index) pairs
// (torch.argmax's order): one wavefront per row.
__global__ __launch_bounds__(256) void wide_argmax_reduce(const float2* __restrict__ parts, int col_tiles, int M,
                                                          int32_t* __restrict__ best) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  float bv = kNegInfW;
  int bi = INT_MAX;
  for (int t = lane; t < col_tiles; t += 64) {
    const float2 p = parts[(int64_t)t * M + row];
    wide_better(bv, bi, p.x, __float_as_int(p.y));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    wide_better(bv, bi, ov, oi);
  }
  if (lane == 0) best[row] = bi == INT_MAX ? -1 : bi;
}

}  // namespace

bool gemm_wide_fits(int M, int N, int K) { return M > 0 && N > 0 && K > 0 && N % kWideTile == 0 && K % kWideChunk == 0; }

// Host checks are the caller's (wptv_gemm): operands 16-byte aligned, leading
// dimensions multiples of 8, operands under 4 GB.
namespace {

constexpr int kWideArgmaxOut = -100;  // launch_wide's out_dtype for the argmax epilogue

template <bool FM>
int launch_wide(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out, int64_t ldo,
                int out_dtype, hipStream_t stream) {
  const int row_tiles = (M + kWideTile - 1) / kWideTile;
  const long long groups = (long long)row_tiles * (N / kWideTile);
  if (groups > 0x7fffffffLL) return fail(WPTV_E_UNSUPPORTED, "gemm: %lld output tiles", groups);
  const auto* xb = static_cast<const unsigned short*>(x);
  const auto* wb = static_cast<const unsigned short*>(w);
  if (out_dtype == kWideArgmaxOut)
    hipLaunchKernelGGL((gemm_wide<kWideArgmax, FM>), dim3((unsigned)groups), dim3(kWideWaves * 64), 0, stream, xb,
                       ldx, wb, ldw, M, N, K, row_tiles, out, ldo);
  else if (out_dtype == WPTV_BF16)
    hipLaunchKernelGGL((gemm_wide<kWideBf16, FM>), dim3((unsigned)groups), dim3(kWideWaves * 64), 0, stream, xb, ldx,
                       wb, ldw, M, N, K, row_tiles, out, ldo);
  else
    hipLaunchKernelGGL((gemm_wide<kWideF32, FM>), dim3((unsigned)groups), dim3(kWideWaves * 64), 0, stream, xb, ldx,
                       wb, ldw, M, N, K, row_tiles, out, ldo);
  return launched("gemm_wide");
}

}  // namespace

int gemm_wide(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out, int64_t ldo,
              int out_dtype, hipStream_t stream) {
  if (!gemm_wide_fits(M, N, K))
    return fail(WPTV_E_UNSUPPORTED, "gemm: the wide product needs N a multiple of %d and K of %d (got %d, %d)",
                kWideTile, kWideChunk, N, K);
  if (ldo % 8) return fail(WPTV_E_INVALID, "gemm: the wide product needs an output leading dimension of 8 elements");
  return launch_wide<false>(x, ldx, w, ldw, M, N, K, out, ldo, out_dtype, stream);
}

}  // namespace wptv

using namespace wptv;

extern "C" int wptv_gemm_fm_wide(const void* x_fm, int x_blocks, const void* w_fm, int M, int N, int K, void* out,
                                 int64_t ldo, int out_dtype, hipStream_t stream) {
  if (!x_fm || !w_fm || !out) return fail(WPTV_E_INVALID, "gemm_fm_wide: x_fm, w_fm and out must be given");
  if (out_dtype != WPTV_BF16 && out_dtype != WPTV_F32)
    return fail(WPTV_E_UNSUPPORTED, "gemm_fm_wide: output dtype %d is neither bf16 nor fp32", out_dtype);
  if (M <= 0 || N <= 0 || K <= 0 || N % kWideTile || K % kWideChunk)
    return fail(WPTV_E_INVALID, "gemm_fm_wide: M > 0, N a multiple of %d and K of %d (got %d, %d, %d)", kWideTile,
                kWideChunk, M, N, K);
  if (x_blocks < fm_row_blocks(M))
    return fail(WPTV_E_INVALID, "gemm_fm_wide: %d row blocks of x hold fewer than M = %d rows", x_blocks, M);
  if (ldo < N || ldo % 8) return fail(WPTV_E_INVALID, "gemm_fm_wide: ldo %lld below N = %d or not a multiple of 8",
                                      (long long)ldo, N);
  if (!aligned(x_fm, 16) || !aligned(w_fm, 16) || !aligned(out, 16))
    return fail(WPTV_E_INVALID, "gemm_fm_wide: x_fm, w_fm and out must be 16-byte aligned");
  if ((double)N * (double)K * 2.0 >= 4.0e9 || (double)x_blocks * 16.0 * (double)K * 2.0 >= 4.0e9)
    return fail(WPTV_E_UNSUPPORTED, "gemm_fm_wide: operands above 4 GB");
  return launch_wide<true>(x_fm, x_blocks, w_fm, N / 16, M, N, K, out, ldo, out_dtype, stream);
}

extern "C" int wptv_gemm_fm_wide_argmax_workspace(int M, int N, size_t* bytes) {
  if (!bytes) return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax_workspace: null output pointer");
  if (M <= 0 || N <= 0 || N % kWideTile)
    return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax_workspace: M > 0 and N a multiple of %d (got %d, %d)", kWideTile,
                M, N);
  *bytes = (size_t)(N / kWideTile) * M * sizeof(float2);
  return WPTV_OK;
}

extern "C" int wptv_gemm_fm_wide_argmax(const void* x_fm, int x_blocks, const void* w_fm, int M, int N, int K,
                                        int32_t* best, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!x_fm || !w_fm || !best || !workspace)
    return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax: x_fm, w_fm, best and workspace must be given");
  if (M <= 0 || N <= 0 || K <= 0 || N % kWideTile || K % kWideChunk)
    return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax: M > 0, N a multiple of %d and K of %d (got %d, %d, %d)",
                kWideTile, kWideChunk, M, N, K);
  if (x_blocks < fm_row_blocks(M))
    return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax: %d row blocks of x hold fewer than M = %d rows", x_blocks, M);
  const size_t need = (size_t)(N / kWideTile) * M * sizeof(float2);
  if (workspace_bytes < need)
    return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (!aligned(x_fm, 16) || !aligned(w_fm, 16) || !aligned(workspace, 16) || !aligned(best, 4))
    return fail(WPTV_E_INVALID, "gemm_fm_wide_argmax: x_fm, w_fm and workspace 16-byte aligned");
  if ((double)N * (double)K * 2.0 >= 4.0e9 || (double)x_blocks * 16.0 * (double)K * 2.0 >= 4.0e9)
    return fail(WPTV_E_UNSUPPORTED, "gemm_fm_wide_argmax: operands above 4 GB");
  int st = launch_wide<true>(x_fm, x_blocks, w_fm, N / 16, M, N, K, workspace, 0, kWideArgmaxOut, stream);
  if (st != WPTV_OK) return st;
  hipLaunchKernelGGL(wide_argmax_reduce, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, stream,
                     static_cast<const float2*>(workspace), N / kWideTile, M, best);
  return launched("wide_argmax_reduce");
}
