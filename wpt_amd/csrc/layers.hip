// The decoder layer's memory-bound pieces around the matrix products, each
// one pass over its rows (the reference's extend runs them as separate torch
// operations: model.py:394-436, attention.py:157-188, layers.py:45-61):
//
//   add_rms_norm  h += delta (the residual add of the sublayer before, when
//                 given), then y = RMSNorm(h) * weight in FP32
//   qkv_post      the exact layer after its q/k/v projection: q = q_norm(q)
//                 per head into (B, T, H, c); the entries [k_norm(k), v] of
//                 each row's first counts[b] tokens appended to the cache
//                 table at start[b] + t (the KV append, cache.py:110-128)
//   swiglu        silu(gate) * up of the feed-forward block's two halves
//
// One wavefront per row (norm) or per (row, head) (q/k norms), every load
// issued before the first use (16-byte vector loads, FP32 sums with wavefront
// reductions); one thread per 8 elements for SwiGLU.
#include "wptv_common.h"

namespace wptv {
namespace {

template <typename T>
struct Vec8;
template <>
struct Vec8<unsigned short> {  // 8 bf16
  typedef unsigned short raw __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ void load(const unsigned short* p, float (&x)[8]) {
    const raw v = *reinterpret_cast<const raw*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bf16_to_f32(v[e]);
  }
  static __device__ __forceinline__ void store(unsigned short* p, const float (&x)[8]) {
    raw v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f32_to_bf16(x[e]);
    *reinterpret_cast<raw*>(p) = v;
  }
  // for an output one later kernel reads once: written non-temporally
  static __device__ __forceinline__ void store_nt(unsigned short* p, const float (&x)[8]) {
    raw v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f32_to_bf16(x[e]);
    __builtin_nontemporal_store(v, reinterpret_cast<raw*>(p));
  }
};
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&x)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = a[e], x[4 + e] = b[e];
  }
  static __device__ __forceinline__ void store(float* p, const float (&x)[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
  static __device__ __forceinline__ void store_nt(float* p, const float (&x)[8]) {
    __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(f32x4{x[4], x[5], x[6], x[7]}, reinterpret_cast<f32x4*>(p + 4));
  }
};

// Values of one row held by a lane: D / 8 / 64 chunks of 8, at most kChunks.
constexpr int kChunks = 8;  // rows up to 64 * 8 * 8 = 4096 wide

// One wavefront (one workgroup) per row: every load of the row -- h, delta
// and the norm weight -- is issued before the first is used (NCH chunks of
// 512 columns, straight-line code: a chunk past the row end re-reads the
// row's last 8 columns and is ignored), so a row costs one memory round
// trip, then the wavefront sum.
template <typename T, int NCH, bool DELTA>
__global__ __launch_bounds__(64) void add_rms_norm(T* __restrict__ h, const T* __restrict__ delta,
                                                   const float* __restrict__ weight, T* __restrict__ y, int M, int D,
                                                   float eps) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  T* hrow = h + (int64_t)row * D;
  const T* drow = DELTA ? delta + (int64_t)row * D : nullptr;
  float x[NCH][8], d[NCH][8], wt[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = min((k * 64 + lane) * 8, D - 8);
    Vec8<T>::load(hrow + col, x[k]);
    if constexpr (DELTA) Vec8<T>::load(drow + col, d[k]);
    Vec8<float>::load(weight + col, wt[k]);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const bool in = (k * 64 + lane) * 8 < D;
    if constexpr (DELTA) {
      // the residual stream keeps the activation dtype, as the reference's h = h + out does
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] = rounded<T>(x[k][e] + d[k][e]);
    }
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part += x[k][e] * x[k][e];
    ss += in ? part : 0.f;
  }
  ss = wave_sum_dpp(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
  T* yrow = y + (int64_t)row * D;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = (k * 64 + lane) * 8;
    if (col < D) {
      if constexpr (DELTA) Vec8<T>::store(hrow + col, x[k]);
      float out[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = x[k][e] * inv * wt[k][e];
      Vec8<T>::store(yrow + col, out);
    }
  }
}

// The first layer's input: h = the embedding rows of the tokens (ids
// outside [0, vocab) read row 0 or vocab - 1; the host checks ids it holds),
// y = RMSNorm(h) * weight, as add_rms_norm without delta; and, when positions
// is given, each token's position lengths[b] + t (row b T + t).
template <typename T, int NCH>
__global__ __launch_bounds__(64) void embed_rms_norm(const int64_t* __restrict__ ids, const T* __restrict__ table,
                                                     int64_t vocab, const float* __restrict__ weight,
                                                     T* __restrict__ h, T* __restrict__ y, int y_blocks, int D,
                                                     float eps, const int64_t* __restrict__ lengths,
                                                     int64_t* __restrict__ positions, int Tn) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  int64_t id = ids[row];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const T* src = table + id * D;
  float x[NCH][8], wt[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = min((k * 64 + lane) * 8, D - 8);
    Vec8<T>::load(src + col, x[k]);
    Vec8<float>::load(weight + col, wt[k]);
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part += x[k][e] * x[k][e];
    ss += (k * 64 + lane) * 8 < D ? part : 0.f;
  }
  ss = wave_sum_dpp(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
  T* hrow = h + (int64_t)row * D;
  T* yrow = y + (int64_t)row * D;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int col = (k * 64 + lane) * 8;
    if (col < D) {
      Vec8<T>::store(hrow + col, x[k]);
      float out[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = x[k][e] * inv * wt[k][e];
      Vec8<T>::store(y_blocks ? y + fm_offset(row, col, y_blocks) : yrow + col, out);
    }
  }
  if (positions && lane == 0) positions[row] = lengths[row / Tn] + row % Tn;
}

// add_rms_norm with delta = the sum of S FP32 parts [S][M][D] (a split-K
// matrix product's parts, summed in a fixed order): one workgroup of D / 8
// threads per row, 8 columns a thread; every load -- the parts, h and the
// norm weight -- issued before the first use.
template <typename T, int S>
__global__ __launch_bounds__(1024) void add_rms_norm_parts(T* __restrict__ h, const float* __restrict__ parts,
                                                           const float* __restrict__ weight, T* __restrict__ y,
                                                           int y_blocks, int M, int D, float eps) {
  __shared__ float wsum[16];
  const int row = blockIdx.x;
  const int col = threadIdx.x * 8;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  T* hrow = h + (int64_t)row * D;
  float x[8], d[S][8], wt[8];
  Vec8<T>::load(hrow + col, x);
#pragma unroll
  for (int z = 0; z < S; ++z) Vec8<float>::load(parts + ((int64_t)z * M + row) * D + col, d[z]);
  Vec8<float>::load(weight + col, wt);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float delta = 0.f;
#pragma unroll
    for (int z = 0; z < S; ++z) delta += d[z][e];
    // the product rounded to the activation dtype, then the residual add in it,
    // as the reference's h = h + out of a bf16 product does
    x[e] = rounded<T>(x[e] + rounded<T>(delta));
    ss += x[e] * x[e];
  }
  ss = wave_sum_dpp(ss);
  if (lane == 0) wsum[wv] = ss;
  __syncthreads();
  float total = 0.f;
  const int waves = (blockDim.x + 63) / 64;
  for (int u = 0; u < waves; ++u) total += wsum[u];
  const float inv = rsqrtf(total / (float)D + eps);
  Vec8<T>::store_nt(hrow + col, x);  // the residual stream: read once, by the next residual add
  float out[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = x[e] * inv * wt[e];
  // y_blocks > 0: y in the fm layout (the next product's operand)
  Vec8<T>::store(y_blocks ? y + fm_offset(row, col, y_blocks) : y + (int64_t)row * D + col, out);
}

// EPL consecutive elements per lane (a head of 64 EPL values per wavefront).
template <typename T, int EPL>
struct Lane {
  static __device__ __forceinline__ void load(const T* p, float (&v)[EPL]) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) v[e] = load_f32(p + e);
  }
  static __device__ __forceinline__ void store(T* p, const float (&v)[EPL]) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) p[e] = from_f32<T>(v[e]);
  }
};
template <int EPL>
struct Lane<unsigned short, EPL> {
  typedef unsigned short raw __attribute__((ext_vector_type(EPL)));
  static __device__ __forceinline__ void load(const unsigned short* p, float (&v)[EPL]) {
    const raw r = *reinterpret_cast<const raw*>(p);
#pragma unroll
    for (int e = 0; e < EPL; ++e) v[e] = bf16_to_f32(r[e]);
  }
  static __device__ __forceinline__ void store(unsigned short* p, const float (&v)[EPL]) {
    raw r;
#pragma unroll
    for (int e = 0; e < EPL; ++e) r[e] = f32_to_bf16(v[e]);
    *reinterpret_cast<raw*>(p) = r;
  }
};
template <>
struct Lane<unsigned short, 1> {
  static __device__ __forceinline__ void load(const unsigned short* p, float (&v)[1]) { v[0] = bf16_to_f32(*p); }
  static __device__ __forceinline__ void store(unsigned short* p, const float (&v)[1]) { *p = f32_to_bf16(v[0]); }
};

// One wavefront per (token row, head) of the H query heads, the key (head
// H) and the value (head H + 1); lane l holds elements EPL l .. EPL l + EPL - 1.
// S > 0: the projection comes as S FP32 split-K parts [S][rows][(H + 2) c]
// (qkv_parts), summed in a fixed order and rounded to T, as the reference's
// bf16 product is.
//
// A window layer (Rope, attention.py:113-135) also turns the last rope.dims
// dimensions of every query head and of the key by the token's position
// start[b] + t (rotate, attention.py:59-71: adjacent pairs (2i, 2i + 1) by
// the angle p / div[i], div[i] = base^(2i / dims), from the normed values in
// T, in FP32) and writes the entry at ring slot (start[b] + t) & ring_mask.
// The divisors come from the host, computed as the reference computes them,
// so that both divide the same numbers.
struct Rope {
  int dims;            // 0: no rotation (an exact layer)
  const float* div;    // [dims / 2]
  uint32_t ring_mask;  // 0: the entry at row start[b] + t (no ring)
};

// The rotation of one head's last `dims` of its C = 64 EPL values, lane l
// holding elements EPL l .. EPL l + EPL - 1: adjacent pairs (2i, 2i + 1) of
// the rotated part turned by the angle pos / div[i], from the values rounded
// to T, in FP32 (attention.py:59-71).  Every lane of the wavefront takes part.
template <typename T, int EPL>
__device__ __forceinline__ void rotate_lane(float (&v)[EPL], int lane, int64_t pos, int dims, const float* div) {
  constexpr int C = 64 * EPL;
  // element d = EPL lane + e; rotated when d >= C - dims, pair i = (d - first) / 2
  const int first = C - dims;
  float mine[EPL], other[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) mine[e] = rounded<T>(v[e]);
  if constexpr (EPL == 1) {
    other[0] = __shfl_xor(mine[0], 1, 64);  // the pair's other element sits on the next lane
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) other[e] = mine[e ^ 1];
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int d = EPL * lane + e;
    if (d < first) continue;
    const int i = (d - first) >> 1;
    const float angle = (float)pos / div[i];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    // (even, odd) -> (even cos - odd sin, even sin + odd cos)
    v[e] = (d & 1) == 0 ? mine[e] * cs - other[e] * sn : other[e] * sn + mine[e] * cs;
  }
}

// The arguments the first loads depend on come first (gfx950 preloads a
// kernel's first 14 argument dwords into SGPRs; the others arrive by a
// scalar load meanwhile).
template <typename T, int EPL, int S>
__global__ __launch_bounds__(256) void qkv_post(int rows, int T_, int H, const float* __restrict__ qkv_parts,
                                                const float* __restrict__ q_norm, const float* __restrict__ k_norm,
                                                const int64_t* __restrict__ start,
                                                const int64_t* __restrict__ counts, float eps,
                                                const T* __restrict__ qkv, int64_t qkv_row, T* __restrict__ q_out,
                                                T* __restrict__ table, int64_t tsb, int64_t tsn, int64_t capacity,
                                                Rope rope) {
  constexpr int C = 64 * EPL;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (gw >= rows * (H + 2)) return;
  const int row = gw / (H + 2), head = gw % (H + 2);
  const int b = row / T_, t = row % T_;
  float v[EPL], wt[EPL];
  if constexpr (S == 0) {
    Lane<T, EPL>::load(qkv + (int64_t)row * qkv_row + (int64_t)head * C + EPL * lane, v);
  } else {
    const int64_t width = (int64_t)(H + 2) * C;
    float d[S][EPL];
#pragma unroll
    for (int z = 0; z < S; ++z) {
      const float* src = qkv_parts + ((int64_t)z * rows + row) * width + (int64_t)head * C + EPL * lane;
#pragma unroll
      for (int e = 0; e < EPL; ++e) d[z][e] = src[e];
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float sum = 0.f;
#pragma unroll
      for (int z = 0; z < S; ++z) sum += d[z][e];
      v[e] = rounded<T>(sum);
    }
  }
  const float* w = (head < H ? q_norm : k_norm) + EPL * lane;  // the value (head H + 1) reads k_norm unused
#pragma unroll
  for (int e = 0; e < EPL; ++e) wt[e] = w[e];
  const int64_t pos = start[b] + t;
  T* dst;
  if (head < H) {
    dst = q_out + ((int64_t)row * H + head) * C;
  } else {
    const int64_t slot = rope.ring_mask ? (pos & (int64_t)rope.ring_mask) : pos;
    if (!(t < counts[b] && pos >= 0 && slot < capacity)) return;
    dst = table + b * tsb + slot * tsn + (head == H ? 0 : C);  // [k_norm(k), v]
  }
  if (head <= H) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss += v[e] * v[e];
    ss = wave_sum_dpp(ss);
    const float inv = rsqrtf(ss / (float)C + eps);
#pragma unroll
    for (int e = 0; e < EPL; ++e) v[e] = v[e] * inv * wt[e];
    if (rope.dims > 0) rotate_lane<T, EPL>(v, lane, pos, rope.dims, rope.div);
  }
  Lane<T, EPL>::store(dst + EPL * lane, v);
}

// RMSNorm of each head of each row: x row r at x + r*row_stride, H heads of
// C = 64 EPL values; out [rows, H, C].  One wavefront per (row, head).  ROPE:
// then each head's last rope_dims values turned by row r's position
// positions[r] (rotate_lane).
template <typename T, int EPL, bool ROPE>
__global__ __launch_bounds__(256) void heads_rms_norm(const T* __restrict__ x, int64_t row_stride,
                                                      const float* __restrict__ weight, T* __restrict__ out, int rows,
                                                      int H, float eps, const int64_t* __restrict__ positions,
                                                      int rope_dims, const float* __restrict__ rope_div) {
  constexpr int C = 64 * EPL;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (gw >= rows * H) return;
  const int row = gw / H, head = gw % H;
  float v[EPL];
  Lane<T, EPL>::load(x + (int64_t)row * row_stride + (int64_t)head * C + EPL * lane, v);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) ss += v[e] * v[e];
  ss = wave_sum_dpp(ss);
  const float inv = rsqrtf(ss / (float)C + eps);
#pragma unroll
  for (int e = 0; e < EPL; ++e) v[e] = v[e] * inv * weight[EPL * lane + e];
  if constexpr (ROPE) rotate_lane<T, EPL>(v, lane, positions[row], rope_dims, rope_div);
  Lane<T, EPL>::store(out + ((int64_t)row * H + head) * C + EPL * lane, v);
}

__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }

template <typename T>
__global__ __launch_bounds__(256) void swiglu(const T* __restrict__ gu, T* __restrict__ out, int M, int F) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= (int64_t)M * F) return;
  const int64_t m = i / F, f = i % F;
  float g[8], u[8], o[8];
  Vec8<T>::load(gu + m * 2 * F + f, g);
  Vec8<T>::load(gu + m * 2 * F + F + f, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = silu(g[e]) * u[e];
  Vec8<T>::store(out + i, o);
}

}  // namespace
}  // namespace wptv

using namespace wptv;

namespace {
bool vec_aligned(const void* p) { return p == nullptr || aligned(p, 16); }
}  // namespace

extern "C" int wptv_add_rms_norm(void* h, const void* delta, const float* weight, void* y, int M, int D, int dtype,
                                 float eps, hipStream_t stream) {
  if (!h || !weight || !y) return fail(WPTV_E_INVALID, "add_rms_norm: h, weight and y must be given");
  if (M < 0 || D <= 0) return fail(WPTV_E_INVALID, "add_rms_norm: bad shape M=%d D=%d", M, D);
  if (D % 8 != 0 || D > 64 * 8 * kChunks)
    return fail(WPTV_E_UNSUPPORTED, "add_rms_norm: width %d is not a multiple of 8 up to %d", D, 64 * 8 * kChunks);
  if (!vec_aligned(h) || !vec_aligned(delta) || !vec_aligned(y))
    return fail(WPTV_E_INVALID, "add_rms_norm: rows must be 16-byte aligned");
  if (M == 0) return WPTV_OK;
  dim3 grid(M);
  const int nch = (D + 511) / 512;
#define WPTV_ARN(TT, NN)                                                                                           \
  do {                                                                                                             \
    if (delta)                                                                                                     \
      hipLaunchKernelGGL((add_rms_norm<TT, NN, true>), grid, dim3(64), 0, stream, static_cast<TT*>(h),             \
                         static_cast<const TT*>(delta), weight, static_cast<TT*>(y), M, D, eps);                   \
    else                                                                                                           \
      hipLaunchKernelGGL((add_rms_norm<TT, NN, false>), grid, dim3(64), 0, stream, static_cast<TT*>(h), nullptr,   \
                         weight, static_cast<TT*>(y), M, D, eps);                                                  \
  } while (0)
#define WPTV_ARN_N(TT)            \
  if (nch <= 1) WPTV_ARN(TT, 1);  \
  else if (nch <= 2) WPTV_ARN(TT, 2); \
  else if (nch <= 4) WPTV_ARN(TT, 4); \
  else WPTV_ARN(TT, 8)
  if (dtype == WPTV_BF16) {
    WPTV_ARN_N(unsigned short);
  } else if (dtype == WPTV_F32) {
    WPTV_ARN_N(float);
  } else {
    return fail(WPTV_E_UNSUPPORTED, "add_rms_norm: dtype %d is neither fp32 nor bf16", dtype);
  }
#undef WPTV_ARN_N
#undef WPTV_ARN
  return launched("add_rms_norm");
}

namespace wptv {
namespace {
// y_blocks > 0: y is an fm operand (bf16, D a multiple of 32, M rows in y_blocks row blocks).
int check_fm_output(const char* what, int y_blocks, int M, int D, int dtype) {
  if (y_blocks == 0) return WPTV_OK;
  if (y_blocks < 0 || dtype != WPTV_BF16 || D % 32 || M > 16 * y_blocks)
    return fail(WPTV_E_INVALID, "%s: an fm output takes bf16, D a multiple of 32 and M <= 16 row blocks (got %d "
                                "row blocks, M %d, D %d)", what, y_blocks, M, D);
  return WPTV_OK;
}
}  // namespace
}  // namespace wptv

extern "C" int wptv_embed_rms_norm(const int64_t* ids, const void* table, int64_t vocab, const float* weight,
                                   void* h, void* y, int y_blocks, int M, int D, int dtype, float eps,
                                   const int64_t* lengths, int64_t* positions, int T, hipStream_t stream) {
  if (!ids || !table || !weight || !h || !y) return fail(WPTV_E_INVALID, "embed_rms_norm: a pointer is missing");
  if (M < 0 || D <= 0 || vocab <= 0) return fail(WPTV_E_INVALID, "embed_rms_norm: bad shape M=%d D=%d", M, D);
  if (positions && (!lengths || T <= 0 || M % T))
    return fail(WPTV_E_INVALID, "embed_rms_norm: positions need lengths and M a multiple of T = %d", T);
  if (D % 8 != 0 || D > 64 * 8 * kChunks)
    return fail(WPTV_E_UNSUPPORTED, "embed_rms_norm: width %d is not a multiple of 8 up to %d", D, 64 * 8 * kChunks);
  if (!vec_aligned(table) || !vec_aligned(h) || !vec_aligned(y))
    return fail(WPTV_E_INVALID, "embed_rms_norm: rows must be 16-byte aligned");
  if (const int st = check_fm_output("embed_rms_norm", y_blocks, M, D, dtype)) return st;
  if (M == 0) return WPTV_OK;
  const int nch = (D + 511) / 512;
#define WPTV_ERN(TT, NN)                                                                                          \
  hipLaunchKernelGGL((embed_rms_norm<TT, NN>), dim3(M), dim3(64), 0, stream, ids, static_cast<const TT*>(table), \
                     vocab, weight, static_cast<TT*>(h), static_cast<TT*>(y), y_blocks, D, eps, lengths,       \
                     positions, T)
#define WPTV_ERN_N(TT)              \
  if (nch <= 1) WPTV_ERN(TT, 1);     \
  else if (nch <= 2) WPTV_ERN(TT, 2); \
  else if (nch <= 4) WPTV_ERN(TT, 4); \
  else WPTV_ERN(TT, 8)
  if (dtype == WPTV_BF16) {
    WPTV_ERN_N(unsigned short);
  } else if (dtype == WPTV_F32) {
    WPTV_ERN_N(float);
  } else {
    return fail(WPTV_E_UNSUPPORTED, "embed_rms_norm: dtype %d is neither fp32 nor bf16", dtype);
  }
#undef WPTV_ERN_N
#undef WPTV_ERN
  return launched("embed_rms_norm");
}

extern "C" int wptv_add_rms_norm_parts(void* h, const float* parts, int splits, const float* weight, void* y,
                                       int y_blocks, int M, int D, int dtype, float eps, hipStream_t stream) {
  if (!h || !parts || !weight || !y) return fail(WPTV_E_INVALID, "add_rms_norm_parts: every pointer must be given");
  if (M < 0 || D <= 0 || splits <= 0)
    return fail(WPTV_E_INVALID, "add_rms_norm_parts: bad shape M=%d D=%d splits=%d", M, D, splits);
  if (D % 8 != 0 || D > 8 * 1024)
    return fail(WPTV_E_UNSUPPORTED, "add_rms_norm_parts: width %d is not a multiple of 8 up to 8192", D);
  if (splits > 8) return fail(WPTV_E_UNSUPPORTED, "add_rms_norm_parts: %d parts above 8", splits);
  if (!vec_aligned(h) || !vec_aligned(parts) || !vec_aligned(y))
    return fail(WPTV_E_INVALID, "add_rms_norm_parts: rows must be 16-byte aligned");
  if (const int st = check_fm_output("add_rms_norm_parts", y_blocks, M, D, dtype)) return st;
  if (M == 0) return WPTV_OK;
  dim3 grid(M), block(D / 8);
#define WPTV_ARNP(TT, SS)                                                                                       \
  hipLaunchKernelGGL((add_rms_norm_parts<TT, SS>), grid, block, 0, stream, static_cast<TT*>(h), parts, weight, \
                     static_cast<TT*>(y), y_blocks, M, D, eps)
#define WPTV_ARNP_S(TT)             \
  switch (splits) {                 \
    case 1: WPTV_ARNP(TT, 1); break; \
    case 2: WPTV_ARNP(TT, 2); break; \
    case 3: WPTV_ARNP(TT, 3); break; \
    case 4: WPTV_ARNP(TT, 4); break; \
    case 5: WPTV_ARNP(TT, 5); break; \
    case 6: WPTV_ARNP(TT, 6); break; \
    case 7: WPTV_ARNP(TT, 7); break; \
    default: WPTV_ARNP(TT, 8); break; \
  }
  if (dtype == WPTV_BF16) {
    WPTV_ARNP_S(unsigned short);
  } else if (dtype == WPTV_F32) {
    WPTV_ARNP_S(float);
  } else {
    return fail(WPTV_E_UNSUPPORTED, "add_rms_norm_parts: dtype %d is neither fp32 nor bf16", dtype);
  }
#undef WPTV_ARNP_S
#undef WPTV_ARNP
  return launched("add_rms_norm_parts");
}

extern "C" int wptv_qkv_post(const void* qkv, int64_t qkv_row_stride, const float* q_norm, const float* k_norm,
                             void* q_out, void* table, int64_t table_stride_b, int64_t table_stride_n,
                             int64_t capacity, const int64_t* start, const int64_t* counts, int B, int T, int H,
                             int c, int dtype, float eps, hipStream_t stream) {
  if (!qkv || !q_norm || !k_norm || !q_out || !table || !start || !counts)
    return fail(WPTV_E_INVALID, "qkv_post: every pointer must be given");
  if (B < 0 || T < 0 || H <= 0 || c <= 0)
    return fail(WPTV_E_INVALID, "qkv_post: bad shape B=%d T=%d H=%d c=%d", B, T, H, c);
  if (c != 64 && c != 128 && c != 256)
    return fail(WPTV_E_UNSUPPORTED, "qkv_post: head width %d is not 64, 128 or 256", c);
  if (qkv_row_stride < (int64_t)(H + 2) * c || table_stride_n < 2 * c)
    return fail(WPTV_E_INVALID, "qkv_post: a row stride below its width");
  const int epl = c / 64;
  const int esize = dtype == WPTV_F32 ? 4 : 2;
  if (qkv_row_stride % epl || table_stride_b % epl || table_stride_n % epl || !aligned(qkv, epl * esize) ||
      !aligned(table, epl * esize) || !aligned(q_out, epl * esize))
    return fail(WPTV_E_INVALID, "qkv_post: rows must be aligned to %d elements", epl);
  if (B == 0 || T == 0) return WPTV_OK;
  const int rows = B * T;
  dim3 grid((unsigned)(((int64_t)rows * (H + 2) + 3) / 4));
#define WPTV_QKV(TT, EE)                                                                                          \
  hipLaunchKernelGGL((qkv_post<TT, EE, 0>), grid, dim3(256), 0, stream, rows, T, H, nullptr, q_norm, k_norm,     \
                     start, counts, eps, static_cast<const TT*>(qkv), qkv_row_stride, static_cast<TT*>(q_out),    \
                     static_cast<TT*>(table), table_stride_b, table_stride_n, capacity, rope)
  const Rope rope{0, nullptr, 0u};
  if (dtype == WPTV_BF16) {
    if (epl == 1) WPTV_QKV(unsigned short, 1);
    else if (epl == 2) WPTV_QKV(unsigned short, 2);
    else WPTV_QKV(unsigned short, 4);
  } else if (dtype == WPTV_F32) {
    if (epl == 1) WPTV_QKV(float, 1);
    else if (epl == 2) WPTV_QKV(float, 2);
    else WPTV_QKV(float, 4);
  } else {
    return fail(WPTV_E_UNSUPPORTED, "qkv_post: dtype %d is neither fp32 nor bf16", dtype);
  }
#undef WPTV_QKV
  return launched("qkv_post");
}

extern "C" int wptv_window_qkv_post(const void* qkv, int64_t qkv_row_stride, const float* q_norm, const float* k_norm,
                                    void* q_out, void* ring, int64_t ring_stride_b, int64_t ring_stride_n,
                                    int ring_rows, const int64_t* start, const int64_t* counts, int B, int T, int H,
                                    int c, int rope_dims, const float* rope_div, int dtype, float eps,
                                    hipStream_t stream) {
  if (!qkv || !q_norm || !k_norm || !q_out || !ring || !start || !counts || (rope_dims > 0 && !rope_div))
    return fail(WPTV_E_INVALID, "window_qkv_post: every pointer must be given");
  if (B < 0 || T < 0 || H <= 0 || c <= 0)
    return fail(WPTV_E_INVALID, "window_qkv_post: bad shape B=%d T=%d H=%d c=%d", B, T, H, c);
  if (c != 64 && c != 128 && c != 256)
    return fail(WPTV_E_UNSUPPORTED, "window_qkv_post: head width %d is not 64, 128 or 256", c);
  if (ring_rows <= 0 || (ring_rows & (ring_rows - 1)) != 0)
    return fail(WPTV_E_INVALID, "window_qkv_post: ring of %d rows is not a power of 2", ring_rows);
  if (rope_dims < 0 || rope_dims > c || rope_dims % 2 != 0)
    return fail(WPTV_E_INVALID, "window_qkv_post: rope dims %d must be even and at most %d", rope_dims, c);
  if (qkv_row_stride < (int64_t)(H + 2) * c || ring_stride_n < 2 * c)
    return fail(WPTV_E_INVALID, "window_qkv_post: a row stride below its width");
  const int epl = c / 64;
  const int esize = dtype == WPTV_F32 ? 4 : 2;
  if (qkv_row_stride % epl || ring_stride_b % epl || ring_stride_n % epl || !aligned(qkv, epl * esize) ||
      !aligned(ring, epl * esize) || !aligned(q_out, epl * esize))
    return fail(WPTV_E_INVALID, "window_qkv_post: rows must be aligned to %d elements", epl);
  if (B == 0 || T == 0) return WPTV_OK;
  const int rows = B * T;
  const Rope rope{rope_dims, rope_div, (uint32_t)(ring_rows - 1)};
  dim3 grid((unsigned)(((int64_t)rows * (H + 2) + 3) / 4));
#define WPTV_WQKV(TT, EE)                                                                                         \
  hipLaunchKernelGGL((qkv_post<TT, EE, 0>), grid, dim3(256), 0, stream, rows, T, H, nullptr, q_norm, k_norm,     \
                     start, counts, eps, static_cast<const TT*>(qkv), qkv_row_stride, static_cast<TT*>(q_out),    \
                     static_cast<TT*>(ring), ring_stride_b, ring_stride_n, (int64_t)ring_rows, rope)
  if (dtype == WPTV_BF16) {
    if (epl == 1) WPTV_WQKV(unsigned short, 1);
    else if (epl == 2) WPTV_WQKV(unsigned short, 2);
    else WPTV_WQKV(unsigned short, 4);
  } else if (dtype == WPTV_F32) {
    if (epl == 1) WPTV_WQKV(float, 1);
    else if (epl == 2) WPTV_WQKV(float, 2);
    else WPTV_WQKV(float, 4);
  } else {
    return fail(WPTV_E_UNSUPPORTED, "window_qkv_post: dtype %d is neither fp32 nor bf16", dtype);
  }
#undef WPTV_WQKV
  return launched("window_qkv_post");
}

extern "C" int wptv_qkv_post_parts(const float* parts, int splits, const float* q_norm, const float* k_norm,
                                   void* q_out, void* table, int64_t table_stride_b, int64_t table_stride_n,
                                   int64_t capacity, const int64_t* start, const int64_t* counts, int B, int T, int H,
                                   int c, int dtype, float eps, hipStream_t stream) {
  if (!parts || !q_norm || !k_norm || !q_out || !table || !start || !counts)
    return fail(WPTV_E_INVALID, "qkv_post_parts: every pointer must be given");
  if (B < 0 || T < 0 || H <= 0 || c <= 0 || splits <= 0)
    return fail(WPTV_E_INVALID, "qkv_post_parts: bad shape B=%d T=%d H=%d c=%d splits=%d", B, T, H, c, splits);
  if (c != 64 && c != 128 && c != 256)
    return fail(WPTV_E_UNSUPPORTED, "qkv_post_parts: head width %d is not 64, 128 or 256", c);
  if (splits > 8) return fail(WPTV_E_UNSUPPORTED, "qkv_post_parts: %d parts above 8", splits);
  if (table_stride_n < 2 * c) return fail(WPTV_E_INVALID, "qkv_post_parts: a row stride below its width");
  const int epl = c / 64;
  const int esize = dtype == WPTV_F32 ? 4 : 2;
  if (table_stride_b % epl || table_stride_n % epl || !aligned(table, epl * esize) || !aligned(q_out, epl * esize) ||
      !aligned(parts, 4 * epl))
    return fail(WPTV_E_INVALID, "qkv_post_parts: rows must be aligned to %d elements", epl);
  if (B == 0 || T == 0) return WPTV_OK;
  const int rows = B * T;
  dim3 grid((unsigned)(((int64_t)rows * (H + 2) + 3) / 4));
#define WPTV_QKVP(TT, EE, SS)                                                                                     \
  hipLaunchKernelGGL((qkv_post<TT, EE, SS>), grid, dim3(256), 0, stream, rows, T, H, parts, q_norm, k_norm, start, \
                     counts, eps, nullptr, 0, static_cast<TT*>(q_out), static_cast<TT*>(table), table_stride_b,   \
                     table_stride_n, capacity, Rope{0, nullptr, 0u})
#define WPTV_QKVP_S(TT, EE)               \
  switch (splits) {                       \
    case 1: WPTV_QKVP(TT, EE, 1); break;  \
    case 2: WPTV_QKVP(TT, EE, 2); break;  \
    case 3: WPTV_QKVP(TT, EE, 3); break;  \
    case 4: WPTV_QKVP(TT, EE, 4); break;  \
    case 5: WPTV_QKVP(TT, EE, 5); break;  \
    case 6: WPTV_QKVP(TT, EE, 6); break;  \
    case 7: WPTV_QKVP(TT, EE, 7); break;  \
    default: WPTV_QKVP(TT, EE, 8); break; \
  }
  if (dtype == WPTV_BF16) {
    if (epl == 1) { WPTV_QKVP_S(unsigned short, 1); }
    else if (epl == 2) { WPTV_QKVP_S(unsigned short, 2); }
    else { WPTV_QKVP_S(unsigned short, 4); }
  } else if (dtype == WPTV_F32) {
    if (epl == 1) { WPTV_QKVP_S(float, 1); }
    else if (epl == 2) { WPTV_QKVP_S(float, 2); }
    else { WPTV_QKVP_S(float, 4); }
  } else {
    return fail(WPTV_E_UNSUPPORTED, "qkv_post_parts: dtype %d is neither fp32 nor bf16", dtype);
  }
#undef WPTV_QKVP_S
#undef WPTV_QKVP
  return launched("qkv_post_parts");
}

namespace {
int heads_norm(const char* what, const void* x, int64_t row_stride, const float* weight, void* out, int rows, int H,
               int c, int dtype, float eps, const int64_t* positions, int rope_dims, const float* rope_div,
               hipStream_t stream) {
  if (!x || !weight || !out) return fail(WPTV_E_INVALID, "%s: every pointer must be given", what);
  if (rows < 0 || H <= 0) return fail(WPTV_E_INVALID, "%s: bad shape rows=%d H=%d", what, rows, H);
  if (c != 64 && c != 128 && c != 256)
    return fail(WPTV_E_UNSUPPORTED, "%s: head width %d is not 64, 128 or 256", what, c);
  if (row_stride < (int64_t)H * c) return fail(WPTV_E_INVALID, "%s: a row stride below H*c", what);
  const bool rope = rope_dims > 0;
  if (rope && (!positions || !rope_div || rope_dims % 2 || rope_dims > c))
    return fail(WPTV_E_INVALID, "%s: the rotation needs positions, divisors and an even width up to %d (got %d)", what,
                c, rope_dims);
  const int epl = c / 64;
  const int esize = dtype == WPTV_F32 ? 4 : 2;
  if (row_stride % epl || !aligned(x, epl * esize) || !aligned(out, epl * esize))
    return fail(WPTV_E_INVALID, "%s: rows must be aligned to %d elements", what, epl);
  if (rows == 0) return WPTV_OK;
  dim3 grid((unsigned)(((int64_t)rows * H + 3) / 4));
#define WPTV_HN(TT, EE)                                                                                             \
  hipLaunchKernelGGL((rope ? heads_rms_norm<TT, EE, true> : heads_rms_norm<TT, EE, false>), grid, dim3(256), 0,     \
                     stream, static_cast<const TT*>(x), row_stride, weight, static_cast<TT*>(out), rows, H, eps,     \
                     positions, rope_dims, rope_div)
  if (dtype == WPTV_BF16) {
    if (epl == 1) WPTV_HN(unsigned short, 1);
    else if (epl == 2) WPTV_HN(unsigned short, 2);
    else WPTV_HN(unsigned short, 4);
  } else if (dtype == WPTV_F32) {
    if (epl == 1) WPTV_HN(float, 1);
    else if (epl == 2) WPTV_HN(float, 2);
    else WPTV_HN(float, 4);
  } else {
    return fail(WPTV_E_UNSUPPORTED, "%s: dtype %d is neither fp32 nor bf16", what, dtype);
  }
#undef WPTV_HN
  return launched(what);
}
}  // namespace

extern "C" int wptv_heads_rms_norm(const void* x, int64_t row_stride, const float* weight, void* out, int rows, int H,
                                   int c, int dtype, float eps, hipStream_t stream) {
  return heads_norm("heads_rms_norm", x, row_stride, weight, out, rows, H, c, dtype, eps, nullptr, 0, nullptr, stream);
}

extern "C" int wptv_heads_rms_norm_rope(const void* x, int64_t row_stride, const float* weight, void* out, int rows,
                                        int H, int c, int dtype, float eps, const int64_t* positions, int rope_dims,
                                        const float* rope_div, hipStream_t stream) {
  return heads_norm("heads_rms_norm_rope", x, row_stride, weight, out, rows, H, c, dtype, eps, positions, rope_dims,
                    rope_div, stream);
}

extern "C" int wptv_swiglu(const void* gate_up, void* out, int M, int F, int dtype, hipStream_t stream) {
  if (!gate_up || !out) return fail(WPTV_E_INVALID, "swiglu: gate_up and out must be given");
  if (M < 0 || F <= 0) return fail(WPTV_E_INVALID, "swiglu: bad shape M=%d F=%d", M, F);
  if (F % 8 != 0) return fail(WPTV_E_UNSUPPORTED, "swiglu: width %d is not a multiple of 8", F);
  if (!vec_aligned(gate_up) || !vec_aligned(out)) return fail(WPTV_E_INVALID, "swiglu: rows must be 16-byte aligned");
  if (M == 0) return WPTV_OK;
  const int64_t threads = (int64_t)M * F / 8;
  dim3 grid((unsigned)((threads + 255) / 256));
  if (dtype == WPTV_BF16)
    hipLaunchKernelGGL(swiglu<unsigned short>, grid, dim3(256), 0, stream, static_cast<const unsigned short*>(gate_up),
                       static_cast<unsigned short*>(out), M, F);
  else if (dtype == WPTV_F32)
    hipLaunchKernelGGL(swiglu<float>, grid, dim3(256), 0, stream, static_cast<const float*>(gate_up),
                       static_cast<float*>(out), M, F);
  else
    return fail(WPTV_E_UNSUPPORTED, "swiglu: dtype %d is neither fp32 nor bf16", dtype);
  return launched("swiglu");
}
