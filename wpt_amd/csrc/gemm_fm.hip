// The verify step's skinny products with fragment-major operands:
//
//   C[M, N] = X[M, K] . W[N, K]^T       bf16 in, FP32 accumulation
//
// the reference's projections under bf16 autocast (attention.py:157-168,
// layers.py:45-61) at M = B (k+1) <= 160 rows.  Both operands are stored in
// the fm layout (wptv_common.h: 1 KiB blocks of 16 rows x 32 columns in the
// register order of v_mfma_f32_16x16x32_bf16): the weights packed once
// (wptv_fm_pack), X written that way by the kernel that produces it (the
// residual add + norm, the attention's output, this file's SwiGLU epilogue).
// So every operand fragment is one 16-byte load per lane from 1 KiB of
// contiguous memory, straight into registers: no LDS staging, no barrier in
// the main loop.
//
// One workgroup of four wavefronts per 16 NB output columns, one part of K
// ("split") and one group of MB row blocks (all of them up to 128 rows; at
// 160 rows each half, 80 rows by twice the columns, which moves less of X and
// W through each compute unit for the same workgroup count: measured on the
// MI355X with cold weights, q/k/v 6.4 against 7.2 us, output 5.7 against 5.9,
// down 10.9 against 12.2, gate/up 18.9 against 20.0; at 320 rows each
// quarter, 80 rows by 128 columns, and 80 by 64 for gate/up); its wavefronts
// share out the part's 32-wide k-steps (wave w takes k-steps w, w + 4, ...),
// each multiplying the group's rows by the NB column blocks:
//
//   C^T[n, m] += W[n, k] . X^T[k, m]    W as the A operand, so lane (j, g)
//                                      ends with columns 4g .. 4g + 3 of row j
//
// with the next k-step's loads in flight while one is multiplied; at the end
// the four wavefronts' sums meet in LDS (added in wave order, a fixed order)
// and the workgroup writes its part (FP32 [split][M][N], summed by the
// consumer: wptv_qkv_post_parts, wptv_add_rms_norm_parts) or, for the
// feed-forward gate/up product, silu(gate) * up in the fm layout the down
// product reads.
//
// Why: at 160 rows a product's workgroups each read all of X for their part of
// K, and that stream, not the weights, bounds them; fm blocks read as
// contiguous KiB run it at twice the rate of row-major X (measured on the
// MI355X: gate/up 21 against 29 us with the same kernel on row-major X).
#include "wptv_common.h"

namespace wptv {
namespace {

constexpr int kFmWaves = 4;
constexpr int kFmDepth = 2;  // k-steps a wavefront has loaded ahead while it multiplies one
constexpr int kFmMaxRows = 320;
enum FmOut { kFmParts = 0, kFmSwiGLU = 1 };

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// One thread per 8 elements of the padded matrix: row r < R copied, padding rows zero.
__global__ __launch_bounds__(256) void fm_pack(const unsigned short* __restrict__ a, int64_t lda, int R, int K,
                                               int rb_count, unsigned short* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int per_row = K / 8;
  if (idx >= (int64_t)rb_count * 16 * per_row) return;
  const int r = (int)(idx / per_row), k = (int)(idx % per_row) * 8;
  u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
  if (r < R) v = *reinterpret_cast<const u16x8*>(a + (int64_t)r * lda + k);
  *reinterpret_cast<u16x8*>(out + fm_offset(r, k, rb_count)) = v;
}

__device__ __forceinline__ unsigned short fm_swiglu_bf16(float g, float u) {
  const float gb = bf16_to_f32(f32_to_bf16(g)), ub = bf16_to_f32(f32_to_bf16(u));
  return f32_to_bf16(gb / (1.f + expf(-gb)) * ub);
}

// grid (N / (16 NB), splits, RBT / MB); split z takes k-steps [4 STEPS z, 4
// STEPS (z + 1)), row group rg the row blocks [MB rg, MB (rg + 1)).  x: RBT
// row blocks; w: NBT = N / 16 row blocks.  OUT kFmParts: part[z][m][n] FP32;
// kFmSwiGLU (NB a multiple of 4, one split): each 4 blocks of a column tile
// are the gate rows of 32 features (2 blocks) then their up rows (2 blocks);
// out holds silu(g) * u [M, N / 2] in the fm layout with RBT row blocks.
template <int MB, int NB, int STEPS, int OUT>
__global__ __launch_bounds__(kFmWaves * 64, 1) void gemm_fm(const u32x4* __restrict__ x, const u32x4* __restrict__ w,
                                                            int NBT, int RBT, int M, int N, void* __restrict__ out) {
  static_assert(OUT != kFmSwiGLU || NB % 4 == 0, "the SwiGLU epilogue pairs two gate and two up blocks");
  constexpr int R = MB * NB * 4;  // accumulator registers per lane
  __shared__ float red[kFmWaves * R * 64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x, z = blockIdx.y, rb0 = blockIdx.z * MB;
  const int ks0 = z * kFmWaves * STEPS + wv;
  const u32x4* wp = w + ((int64_t)ks0 * NBT + tile * NB) * 64 + lane;
  const u32x4* xp = x + ((int64_t)ks0 * RBT + rb0) * 64 + lane;
  const int64_t wstep = (int64_t)kFmWaves * NBT * 64, xstep = (int64_t)kFmWaves * RBT * 64;

  f32x4 acc[MB][NB];
#pragma unroll
  for (int rb = 0; rb < MB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[rb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 wb[kFmDepth][NB], xb[kFmDepth][MB];
  // Step s multiplies k-step s - kFmDepth, then loads k-step s.  The
  // scheduling barriers keep the loads where they are written (the compiler
  // would otherwise sink them next to their use, one memory latency a step).
#pragma unroll
  for (int s = 0; s < STEPS + kFmDepth; ++s) {
    if (s >= kFmDepth) {
      const int d = (s - kFmDepth) % kFmDepth;
#pragma unroll
      for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wb[d][nb]),
                                                                __builtin_bit_cast(bf16x8, xb[d][rb]), acc[rb][nb], 0,
                                                                0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (s < STEPS) {
      const int d = s % kFmDepth;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) wb[d][nb] = wp[s * wstep + nb * 64];
#pragma unroll
      for (int rb = 0; rb < MB; ++rb) xb[d][rb] = xp[s * xstep + rb * 64];
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // the four wavefronts' sums: red[wave][register][lane], added in wave order
#pragma unroll
  for (int rb = 0; rb < MB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(wv * R + (rb * NB + nb) * 4 + i) * 64 + lane] = acc[rb][nb][i];
  __syncthreads();
  auto summed = [&](int pair, int i) {
    float s = red[(0 * R + pair * 4 + i) * 64 + lane];
#pragma unroll
    for (int u = 1; u < kFmWaves; ++u) s += red[(u * R + pair * 4 + i) * 64 + lane];
    return s;
  };
  const int j = lane & 15, g = lane >> 4;
  if constexpr (OUT == kFmParts) {
    for (int p = wv; p < MB * NB; p += kFmWaves) {
      const int rb = p / NB, nb = p % NB;
      const int m = (rb0 + rb) * 16 + j;
      if (m >= M) continue;
      const f32x4 v = {summed(p, 0), summed(p, 1), summed(p, 2), summed(p, 3)};
      // the parts are read once, by the consumer kernel: written non-temporally
      __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(static_cast<float*>(out) + ((int64_t)z * M + m) * N +
                                                              tile * NB * 16 + nb * 16 + 4 * g));
    }
  } else {
    typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
    // output block p: row block rb, gate block gb (of the tile's NB / 2), feature column 16 gb + 4 g
    constexpr int kOutBlocks = NB / 2;
    for (int p = wv; p < MB * kOutBlocks; p += kFmWaves) {
      const int rb = p / kOutBlocks, gb = p % kOutBlocks;
      const int m = (rb0 + rb) * 16 + j;
      if (m >= M) continue;
      const int nb = 4 * (gb >> 1) + (gb & 1);  // the gate block; its up block is nb + 2
      const int pg = rb * NB + nb, pu = pg + 2;
      u16x4 res;
#pragma unroll
      for (int i = 0; i < 4; ++i) res[i] = fm_swiglu_bf16(summed(pg, i), summed(pu, i));
      *reinterpret_cast<u16x4*>(static_cast<unsigned short*>(out) + fm_offset(m, tile * 8 * NB + gb * 16 + 4 * g, RBT)) =
          res;
    }
  }
}

// k-steps per wavefront the kernel is built for
constexpr int kFmSteps[] = {2, 4, 8, 11, 16};

bool fm_steps_built(int s) {
  for (int v : kFmSteps)
    if (v == s) return true;
  return false;
}

struct FmPlan {
  int mb, nb, splits, steps;
  int groups;  // row groups of mb row blocks: 2 at 160 rows, 4 at 320, else 1
  size_t bytes;
};

int fm_plan(int M, int N, int K, bool swiglu, int requested, FmPlan* p) {
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(WPTV_E_INVALID, "gemm_fm: M, N and K must be positive (got %d, %d, %d)", M, N, K);
  if (M > kFmMaxRows) return fail(WPTV_E_UNSUPPORTED, "gemm_fm: M = %d above %d rows", M, kFmMaxRows);
  const int nb = swiglu ? 4 : 2;
  if (N % (16 * nb) || K % (32 * kFmWaves))
    return fail(WPTV_E_UNSUPPORTED, "gemm_fm: N (%d) must be a multiple of %d and K (%d) of %d", N, 16 * nb, K,
                32 * kFmWaves);
  const int quarter = K / (32 * kFmWaves);  // k-steps per wavefront over the whole of K
  const int tiles = N / (16 * nb);
  int s = 0;
  if (swiglu) {
    if (requested > 1) return fail(WPTV_E_INVALID, "gemm_fm: the SwiGLU product takes one part of K");
    s = 1;
    if (!fm_steps_built(quarter))
      return fail(WPTV_E_UNSUPPORTED, "gemm_fm: K = %d gives %d k-steps per wavefront, which no kernel form takes",
                  K, quarter);
  } else if (requested > 0) {
    if (quarter % requested || !fm_steps_built(quarter / requested) || requested > 8)
      return fail(WPTV_E_UNSUPPORTED, "gemm_fm: %d parts of K = %d have no kernel form", requested, K);
    s = requested;
  } else {
    // the most parts that keep one workgroup per compute unit, else the
    // fewest (measured in the step at 160 rows: q/k/v 10.0 us in 2 parts of
    // 144 workgroups, 11.2 us in 4 parts of 288)
    const int cus = compute_units();
    int fewest = 0;
    for (int c = 1; c <= 8; ++c) {
      if (quarter % c || !fm_steps_built(quarter / c)) continue;
      if (!fewest) fewest = c;
      if (tiles * c <= cus) s = c;
    }
    if (!s) s = fewest;
    if (!s) return fail(WPTV_E_UNSUPPORTED, "gemm_fm: no part count of K = %d has a kernel form", K);
  }
  // row groups: the same workgroups as all rows by nb blocks, squarer tiles
  const int rb = fm_row_blocks(M);
  p->mb = rb;
  p->nb = nb;
  p->groups = 1;
  if (rb == 10 && N % (32 * nb) == 0) {  // 160 rows: halves by 2 nb blocks
    p->mb = 5;
    p->nb = 2 * nb;
    p->groups = 2;
  } else if (rb == 20 && N % (64 * nb) == 0) {  // 320 rows: quarters by 4 nb blocks (gate/up: by nb, two per CU)
    p->mb = 5;
    p->nb = swiglu ? nb : 4 * nb;
    p->groups = 4;
  } else if (rb > 10) {
    return fail(WPTV_E_UNSUPPORTED, "gemm_fm: %d rows have no kernel form (up to 160, or 289 to 320)", M);
  }
  p->splits = s;
  p->steps = quarter / s;
  p->bytes = swiglu ? 0 : align_up((size_t)s * M * N * sizeof(float), 256);
  return WPTV_OK;
}

template <int MB, int NB, int OUT>
int launch_fm_steps(int steps, dim3 grid, hipStream_t stream, const void* x, const void* w, int NBT, int RBT, int M,
                    int N, void* out) {
  const auto* xv = static_cast<const u32x4*>(x);
  const auto* wv = static_cast<const u32x4*>(w);
#define WPTV_FM(SS)                                                                                                \
  hipLaunchKernelGGL((gemm_fm<MB, NB, SS, OUT>), grid, dim3(kFmWaves * 64), 0, stream, xv, wv, NBT, RBT, M, N, \
                     out)
  switch (steps) {
    case 2: WPTV_FM(2); break;
    case 4: WPTV_FM(4); break;
    case 8: WPTV_FM(8); break;
    case 11: WPTV_FM(11); break;
    case 16: WPTV_FM(16); break;
    default: return fail(WPTV_E_UNSUPPORTED, "gemm_fm: %d k-steps per wavefront have no kernel form", steps);
  }
#undef WPTV_FM
  return launched("gemm_fm");
}

template <int NB, int OUT>
int launch_fm(const FmPlan& p, hipStream_t stream, const void* x, const void* w, int M, int N, void* out) {
  const int NBT = N / 16, RBT = fm_row_blocks(M);
  const dim3 grid(N / (16 * p.nb), p.splits, p.groups);
  if (p.groups > 1) {  // groups of 5 row blocks by 4 or 8 column blocks
    if (p.nb == 4) return launch_fm_steps<5, 4, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
    return launch_fm_steps<5, 8, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
  }
  switch (p.mb) {
    case 2: return launch_fm_steps<2, NB, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
    case 4: return launch_fm_steps<4, NB, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
    case 6: return launch_fm_steps<6, NB, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
    case 8: return launch_fm_steps<8, NB, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
    default: return launch_fm_steps<10, NB, OUT>(p.steps, grid, stream, x, w, NBT, RBT, M, N, out);
  }
}

bool fm_operands_ok(const void* x, const void* w, int N, int K) {
  return aligned(x, 16) && aligned(w, 16) && (double)N * (double)K * 2.0 < 4.0e9;
}

}  // namespace
}  // namespace wptv

using namespace wptv;

extern "C" int wptv_fm_pack(const void* a, int64_t lda, int rows, int K, int row_blocks, void* out,
                            hipStream_t stream) {
  if (!a || !out) return fail(WPTV_E_INVALID, "fm_pack: a and out must be given");
  if (rows < 0 || K <= 0 || K % 32 || row_blocks < 0 || rows > 16 * row_blocks)
    return fail(WPTV_E_INVALID, "fm_pack: %d rows of K = %d (a multiple of 32) in %d row blocks of 16", rows, K,
                row_blocks);
  if (lda < K || lda % 8 || !aligned(a, 16) || !aligned(out, 16))
    return fail(WPTV_E_INVALID, "fm_pack: a and out 16-byte aligned, lda >= K and a multiple of 8");
  const long long items = (long long)row_blocks * 16 * (K / 8);
  if (items == 0) return WPTV_OK;
  hipLaunchKernelGGL(fm_pack, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const unsigned short*>(a), lda, rows, K, row_blocks,
                     static_cast<unsigned short*>(out));
  return launched("fm_pack");
}

extern "C" int wptv_fm_row_blocks(int M) { return fm_row_blocks(M); }

extern "C" int wptv_gemm_fm_plan(int M, int N, int K, int swiglu, int* splits, size_t* parts_bytes) {
  if (!splits || !parts_bytes) return fail(WPTV_E_INVALID, "gemm_fm_plan: null output pointer");
  FmPlan p;
  const int st = fm_plan(M, N, K, swiglu != 0, *splits, &p);
  if (st != WPTV_OK) return st;
  *splits = p.splits;
  *parts_bytes = p.bytes;
  return WPTV_OK;
}

extern "C" int wptv_gemm_fm_parts(const void* x_fm, const void* w_fm, int M, int N, int K, int splits, float* parts,
                                  size_t parts_bytes, hipStream_t stream) {
  if (!x_fm || !w_fm || !parts) return fail(WPTV_E_INVALID, "gemm_fm_parts: x, w and parts must be given");
  FmPlan p;
  const int st = fm_plan(M, N, K, false, splits, &p);
  if (st != WPTV_OK) return st;
  if (splits <= 0) return fail(WPTV_E_INVALID, "gemm_fm_parts: take the part count from wptv_gemm_fm_plan");
  if (!fm_operands_ok(x_fm, w_fm, N, K) || !aligned(parts, 16))
    return fail(WPTV_E_INVALID, "gemm_fm_parts: x, w and parts 16-byte aligned, w under 4 GB");
  const size_t need = (size_t)p.splits * M * N * sizeof(float);
  if (parts_bytes < need) return fail(WPTV_E_INVALID, "gemm_fm_parts: %zu bytes of parts, %zu needed", parts_bytes, need);
  return launch_fm<2, kFmParts>(p, stream, x_fm, w_fm, M, N, parts);
}

extern "C" int wptv_gemm_fm_swiglu(const void* x_fm, const void* w_fm, int M, int N, int K, void* out_fm,
                                   hipStream_t stream) {
  if (!x_fm || !w_fm || !out_fm) return fail(WPTV_E_INVALID, "gemm_fm_swiglu: x, w and out must be given");
  FmPlan p;
  const int st = fm_plan(M, N, K, true, 1, &p);
  if (st != WPTV_OK) return st;
  if (!fm_operands_ok(x_fm, w_fm, N, K) || !aligned(out_fm, 8))
    return fail(WPTV_E_INVALID, "gemm_fm_swiglu: x and w 16-byte aligned (out 8), w under 4 GB");
  return launch_fm<4, kFmSwiGLU>(p, stream, x_fm, w_fm, M, N, out_fm);
}
