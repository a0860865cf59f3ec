// Exact attention's choice of rows for gfx950: for each query, the top_k
// table rows it weighs most among those at least `window` tokens back
// (HySparse's oracle selection), which the sparse layers after an exact
// layer read.
//
// Semantics follow the reference's PyTorch form
// (packages/wpt-model/src/wpt_model/pytorch_kernels.py:112-117): a row's
// score for a query is its largest log-weight over the heads,
//   score(n) = max_h (q_h . k_n * scale - lse_h),
// lse_h the head's log-sum-exp over every row the query sees; the rows
// n > p - window are not candidates; the query keeps the K highest-scoring
// candidates, K = max(0, min(top_k, N - window)), or every candidate and -1
// after them when it has fewer.  The reference leaves the order of equal
// scores to torch.topk ("whichever row topk returns first"); here the rows
// strictly above the K-th largest score come first in row order, then the
// rows equal to it, lowest rows first, up to K.
//
// Two passes (the Triton kernel instead re-streams the keys in up to 16
// counting passes, triton_kernels.py:393-508):
//   choice_scores_*  one workgroup per (batch row, block of query positions,
//                    64 table rows): the scores of the 64 rows for every
//                    query of the block, written once (4 bytes per row and
//                    query, against the 2c bytes of the key read once)
//                      bf16, head width 64 or 128: S^T = K . Q^T on
//                        v_mfma_f32_16x16x32_bf16 (one key row per lane as
//                        the A operand), the max over heads through LDS
//                      otherwise: FP32 dot products on the VALU
//   choice_select_regs  one workgroup per query, tables up to 8192 rows: the
//                    query's scores in registers, the K-th largest found two
//                    bits at a time with packed workgroup counts, the chosen
//                    rows written in row order after one exclusive scan
//   choice_select    longer tables: a 4-pass radix select of the K-th
//                    largest score (order-preserving keys, most significant
//                    byte first; the scores stay in L2), then one pass that
//                    compacts the chosen rows in row order with wavefront
//                    ballots
#include "wptv_common.h"

namespace wptv {
namespace {

constexpr int kKeys = 64;       // table rows per score workgroup
constexpr int kMaxRows = 128;   // query rows (positions x heads) per score workgroup
constexpr int kST = 256;        // threads of the score and select kernels
constexpr float kInf = __builtin_inff();

// The candidates of query position p: rows 0 .. far - 1.
__device__ __forceinline__ int far_rows(int64_t p, int window, int N) {
  int64_t f = p - window + 1;
  f = f < N ? f : N;
  return f > 0 ? (int)f : 0;
}

// Workgroup coordinates of the score kernels: (batch row, position block,
// row block); the first position of the block and its count.
struct ScoreBlock {
  int b, t0, tn, n0;
};

__device__ __forceinline__ ScoreBlock score_block(int T, int tb_positions, int ntb, int nkb) {
  ScoreBlock s;
  const int kb = blockIdx.x % nkb;
  const int rest = blockIdx.x / nkb;
  s.b = rest / ntb;
  s.t0 = (rest % ntb) * tb_positions;
  s.tn = min(tb_positions, T - s.t0);
  s.n0 = kb * kKeys;
  return s;
}

// Rows past every query's candidates of the block are never read: such a
// row block writes nothing.
__device__ __forceinline__ bool block_has_candidates(const ScoreBlock& s, const int64_t* pos_b, int window, int N) {
  int far = 0;
  for (int t = 0; t < s.tn; ++t) far = max(far, far_rows(pos_b[s.t0 + t], window, N));
  return s.n0 < far;
}

// xs[key][r] holds q_r . k_key * scale - lse_r in log2 units for the block's
// R = tn * H query rows; each (row, position) takes the max over the heads.
__device__ __forceinline__ void store_scores(const float (*xs)[kMaxRows + 1], const ScoreBlock& s,
                                             const int64_t* pos_b, int T, int H, int N, int window,
                                             float* __restrict__ scores, int64_t ns) {
  for (int idx = threadIdx.x; idx < kKeys * s.tn; idx += kST) {
    const int key = idx % kKeys, t = idx / kKeys;
    const int n = s.n0 + key;
    if (n >= N) continue;
    float m = -kInf;
    for (int h = 0; h < H; ++h) m = fmaxf(m, xs[key][t * H + h]);
    const int64_t p = pos_b[s.t0 + t];
    scores[((int64_t)s.b * T + s.t0 + t) * ns + n] = (int64_t)n <= p - window ? m : -kInf;
  }
}

template <int C>
__global__ __launch_bounds__(kST) void choice_scores_mfma(
    const unsigned short* __restrict__ q, const unsigned short* __restrict__ k, int64_t ksb, int64_t ksn,
    const int64_t* __restrict__ positions, const float* __restrict__ lse, int T, int H, int N, int window,
    float scale_log2, int tb_positions, int ntb, int nkb, float* __restrict__ scores, int64_t ns) {
  constexpr int S = C / 32;  // k-steps of 16x16x32
  __shared__ float xs[kKeys][kMaxRows + 1];
  const ScoreBlock blk = score_block(T, tb_positions, ntb, nkb);
  const int64_t* pos_b = positions + (int64_t)blk.b * T;
  if (!block_has_candidates(blk, pos_b, window, N)) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int R = blk.tn * H;

  // A operand: key row n0 + 16 w + j (clamped; the clamped rows are not
  // written), elements 32 s + 8 g .. + 7 of k-step s.
  int n = blk.n0 + 16 * w + j;
  n = n < N ? n : N - 1;
  const unsigned short* krow = k + (int64_t)blk.b * ksb + (int64_t)n * ksn;
  bf16x8 kop[S];
#pragma unroll
  for (int s = 0; s < S; ++s) kop[s] = *reinterpret_cast<const bf16x8*>(krow + 32 * s + 8 * g);

  // B operand: query row 16 mb + j of the block (padding rows repeat the
  // last; their scores are never read).
  const unsigned short* qb = q + ((int64_t)blk.b * T + blk.t0) * H * C;
  const float* lb = lse + ((int64_t)blk.b * T + blk.t0) * H;
  const int MB = (R + 15) / 16;
  for (int mb = 0; mb < MB; ++mb) {
    const int r = 16 * mb + j;
    const int rr = r < R ? r : R - 1;
    bf16x8 qop[S];
#pragma unroll
    for (int s = 0; s < S; ++s) qop[s] = *reinterpret_cast<const bf16x8*>(qb + (int64_t)rr * C + 32 * s + 8 * g);
    const float l2 = lb[rr] * kLog2e;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[s], qop[s], acc, 0, 0, 0);
    // acc[i] = S^T[key 4 g + i][query row r]
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[16 * w + 4 * g + i][r] = fmaf(acc[i], scale_log2, -l2);
  }
  __syncthreads();
  store_scores(xs, blk, pos_b, T, H, N, window, scores, ns);
}

// 16 heads (each position's heads are one 16-row MFMA block, so the max over
// the heads is a reduction over the 16 lanes of a lane group): one
// workgroup per (batch row, 512 table rows), every position of the pass.
// Each wavefront takes 128 rows in sub-blocks of 16, the keys of four
// sub-blocks loaded before the first is used, the queries held in
// registers for the whole range.
constexpr int kH16Rows = 512;  // table rows per workgroup
constexpr int kH16Batch = 4;   // 16-row sub-blocks whose keys are in flight together

template <int C, int TT>
__global__ __launch_bounds__(kST) void choice_scores_h16(
    const unsigned short* __restrict__ q, const unsigned short* __restrict__ k, int64_t ksb, int64_t ksn,
    const int64_t* __restrict__ positions, const float* __restrict__ lse, int T, int N, int window, float scale_log2,
    int nkb, float* __restrict__ scores, int64_t ns) {
  constexpr int S = C / 32;
  const int b = blockIdx.x / nkb;
  const int n0 = (blockIdx.x % nkb) * kH16Rows;
  const int64_t* pos_b = positions + (int64_t)b * T;
  int far = 0;
  for (int t = 0; t < T; ++t) far = max(far, far_rows(pos_b[t], window, N));
  if (n0 >= far) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  bf16x8 qop[TT][S];
  float l2[TT];
  int64_t lim[TT];  // row n is a candidate of position t iff n <= lim[t]
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tt = t < T ? t : T - 1;
    const unsigned short* qrow = q + (((int64_t)b * T + tt) * 16 + j) * C;
#pragma unroll
    for (int s = 0; s < S; ++s) qop[t][s] = *reinterpret_cast<const bf16x8*>(qrow + 32 * s + 8 * g);
    l2[t] = lse[((int64_t)b * T + tt) * 16 + j] * kLog2e;
    lim[t] = pos_b[tt] - window;
  }
  const int wn0 = n0 + w * (kH16Rows / 4);
  const unsigned short* kb = k + (int64_t)b * ksb;
#pragma unroll 1
  for (int sb0 = 0; sb0 < kH16Rows / 4 / 16; sb0 += kH16Batch) {
    if (wn0 + 16 * sb0 >= far) break;
    bf16x8 kop[kH16Batch][S];
#pragma unroll
    for (int u = 0; u < kH16Batch; ++u) {
      int n = wn0 + 16 * (sb0 + u) + j;
      n = n < N ? n : N - 1;  // clamped rows are not written
#pragma unroll
      for (int s = 0; s < S; ++s) kop[u][s] = *reinterpret_cast<const bf16x8*>(kb + (int64_t)n * ksn + 32 * s + 8 * g);
    }
#pragma unroll
    for (int u = 0; u < kH16Batch; ++u) {
      const int nb = wn0 + 16 * (sb0 + u);  // the sub-block's first row
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= T) break;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < S; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[u][s], qop[t][s], acc, 0, 0, 0);
        // acc[i] = S^T[row nb + 4g + i][head j]; the max over the 16 heads
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = row16_max(fmaf(acc[i], scale_log2, -l2[t]));
        // lane j < 4 writes row nb + 4g + j: 16 consecutive rows per sub-block
        const int n = nb + 4 * g + j;
        if (j < 4 && n < N) {
          const float v = j == 0 ? x[0] : j == 1 ? x[1] : j == 2 ? x[2] : x[3];
          scores[((int64_t)b * T + t) * ns + n] = (int64_t)n <= lim[t] ? v : -kInf;
        }
      }
    }
  }
}

template <typename E>
__global__ __launch_bounds__(kST) void choice_scores_generic(
    const E* __restrict__ q, const E* __restrict__ k, int64_t ksb, int64_t ksn, const int64_t* __restrict__ positions,
    const float* __restrict__ lse, int T, int H, int c, int N, int window, float scale_log2, int tb_positions,
    int ntb, int nkb, float* __restrict__ scores, int64_t ns) {
  __shared__ float xs[kKeys][kMaxRows + 1];
  __shared__ float ks[kKeys][256 + 1];
  const ScoreBlock blk = score_block(T, tb_positions, ntb, nkb);
  const int64_t* pos_b = positions + (int64_t)blk.b * T;
  if (!block_has_candidates(blk, pos_b, window, N)) return;
  const int R = blk.tn * H;
  for (int idx = threadIdx.x; idx < kKeys * c; idx += kST) {
    const int key = idx / c, e = idx % c;
    const int n = min(blk.n0 + key, N - 1);
    ks[key][e] = load_f32(k + (int64_t)blk.b * ksb + (int64_t)n * ksn + e);
  }
  __syncthreads();
  const E* qb = q + ((int64_t)blk.b * T + blk.t0) * H * c;
  const float* lb = lse + ((int64_t)blk.b * T + blk.t0) * H;
  // lanes of a wavefront share the query row (uniform loads) and take 64 keys
  for (int idx = threadIdx.x; idx < kKeys * R; idx += kST) {
    const int key = idx % kKeys, r = idx / kKeys;
    const E* qr = qb + (int64_t)r * c;
    float d = 0.f;
    for (int e = 0; e < c; ++e) d = fmaf(load_f32(qr + e), ks[key][e], d);
    xs[key][r] = fmaf(d, scale_log2, -lb[r] * kLog2e);
  }
  __syncthreads();
  store_scores(xs, blk, pos_b, T, H, N, window, scores, ns);
}

__global__ __launch_bounds__(kST) void choice_select(const float* __restrict__ scores, int64_t ns,
                                                     const int64_t* __restrict__ positions, int N, int window, int K,
                                                     int64_t* __restrict__ chosen) {
  __shared__ int hist[256];
  __shared__ int sel[2];
  __shared__ int wcount[2][kST / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t bt = blockIdx.x;
  const int nf = far_rows(positions[bt], window, N);
  int64_t* out = chosen + bt * K;
  const float* s = scores + bt * ns;
  if (nf <= K) {  // every candidate, then none
    for (int i = tid; i < K; i += kST) out[i] = i < nf ? i : -1;
    return;
  }
  // The K-th largest key.
  uint32_t prefix = 0, mask = 0;
  int remaining = K;
  for (int shift = 24; shift >= 0; shift -= 8) {
    __syncthreads();
    hist[tid] = 0;
    __syncthreads();
    for (int n = tid; n < nf; n += kST) {
      const uint32_t u = order_key(s[n]);
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid < 64) {
      // lane l holds bins 4l .. 4l + 3; suffix = entries in bins >= 4l
      int cnt[4], total = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) total += (cnt[e] = hist[4 * lane + e]);
      int suffix = total;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int other = __shfl_down(suffix, o, 64);
        if (lane + o < 64) suffix += other;
      }
      const uint64_t hit = __builtin_amdgcn_ballot_w64(suffix >= remaining);
      const int top = 63 - __builtin_clzll(hit);  // the highest lane still reaching the K-th entry
      if (lane == top) {
        int above = suffix - total;
        int digit = 4 * lane;
        for (int e = 3; e >= 0; --e) {
          if (above + cnt[e] >= remaining) {
            digit = 4 * lane + e;
            break;
          }
          above += cnt[e];
        }
        sel[0] = digit;
        sel[1] = remaining - above;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sel[0] << shift;
    mask |= 255u << shift;
    remaining = sel[1];
  }
  // Rows above the K-th largest (K - remaining of them), then `remaining`
  // rows equal to it, each in row order.
  const uint32_t tau = prefix;
  const int need_eq = remaining, n_gt = K - remaining;
  const uint64_t below = (1ull << lane) - 1ull;
  int base_gt = 0, base_eq = 0;
  for (int start = 0; start < nf; start += kST) {
    const int n = start + tid;
    const uint32_t u = n < nf ? order_key(s[n]) : 0u;
    const bool gt = n < nf && u > tau, eq = n < nf && u == tau;
    const uint64_t bg = __builtin_amdgcn_ballot_w64(gt), be = __builtin_amdgcn_ballot_w64(eq);
    if (lane == 0) {
      wcount[0][w] = __builtin_popcountll(bg);
      wcount[1][w] = __builtin_popcountll(be);
    }
    __syncthreads();
    int pg = base_gt, pe = base_eq;
    for (int i = 0; i < w; ++i) {
      pg += wcount[0][i];
      pe += wcount[1][i];
    }
    pg += __builtin_popcountll(bg & below);
    pe += __builtin_popcountll(be & below);
    if (gt) out[pg] = n;
    if (eq && pe < need_eq) out[n_gt + pe] = n;
#pragma unroll
    for (int i = 0; i < kST / 64; ++i) {
      base_gt += wcount[0][i];
      base_eq += wcount[1][i];
    }
    __syncthreads();
    if (base_gt >= n_gt && base_eq >= need_eq) break;  // uniform: every thread holds the same counts
  }
}

// Sum over the workgroup, one barrier: red holds two buffers of one value per
// wavefront, used in turn (a wavefront writes a round's buffer only after
// every wavefront has passed the barrier of the round before, and so has read
// the buffer of two rounds before).
__device__ __forceinline__ uint64_t block_sum_u64(uint32_t lo, uint32_t hi, uint64_t (*red)[kST / 64], int round) {
  const uint64_t x = (uint64_t)wave_sum_u32(lo) | ((uint64_t)wave_sum_u32(hi) << 32);
  if ((threadIdx.x & 63) == 0) red[round & 1][threadIdx.x >> 6] = x;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < kST / 64; ++i) r += red[round & 1][i];
  return r;
}

// The select for up to kST * ITEMS candidates: thread t holds the keys of
// rows ITEMS t .. ITEMS t + ITEMS - 1 in registers (one memory round trip);
// the K-th largest key is found two bits at a time from the top (16 rounds,
// each counting the keys at or above three candidates in one packed
// reduction), and the chosen rows are written in row order after one
// exclusive scan of the threads' counts.
template <int ITEMS>
__global__ __launch_bounds__(kST) void choice_select_regs(const float* __restrict__ scores, int64_t ns,
                                                          const int64_t* __restrict__ positions, int N, int window,
                                                          int K, int64_t* __restrict__ chosen) {
  static_assert(ITEMS % 4 == 0 && kST * ITEMS <= 65535, "packed counts hold 16 bits");
  __shared__ uint64_t red[2][kST / 64];
  __shared__ int scan_g[kST / 64], scan_e[kST / 64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t bt = blockIdx.x;
  const int nf = far_rows(positions[bt], window, N);
  int64_t* out = chosen + bt * K;
  if (nf <= K) {  // every candidate, then none
    for (int i = tid; i < K; i += kST) out[i] = i < nf ? i : -1;
    return;
  }
  const float* s = scores + bt * ns;
  const int base = tid * ITEMS;
  uint32_t key[ITEMS];  // 0 (below every score's key) past the candidates
#pragma unroll
  for (int v4 = 0; v4 < ITEMS / 4; ++v4) {
    const int n = base + 4 * v4;
    const f32x4 x = n < nf ? *reinterpret_cast<const f32x4*>(s + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) key[4 * v4 + e] = n + e < nf ? order_key(x[e]) : 0u;
  }
  // the largest t with at least K keys >= t: the K-th largest key
  uint32_t prefix = 0;
  for (int shift = 30, round = 0; shift >= 0; shift -= 2, ++round) {
    const uint32_t c1 = prefix | (1u << shift), c2 = prefix | (2u << shift), c3 = prefix | (3u << shift);
    uint32_t n12 = 0, n3 = 0;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      n12 += (key[i] >= c1 ? 1u : 0u) + (key[i] >= c2 ? 65536u : 0u);
      n3 += key[i] >= c3 ? 1u : 0u;
    }
    const uint64_t sum = block_sum_u64(n12, n3, red, round);
    const int s1 = (int)(sum & 65535), s2 = (int)((sum >> 16) & 65535), s3 = (int)(sum >> 32);
    prefix = s3 >= K ? c3 : s2 >= K ? c2 : s1 >= K ? c1 : prefix;
  }
  const uint32_t tau = prefix;
  int cg = 0, ce = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    cg += key[i] > tau ? 1 : 0;
    ce += key[i] == tau ? 1 : 0;
  }
  // exclusive scan of (cg, ce) over the threads in row order
  int ig = cg, ie = ce;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int og = __shfl_up(ig, o, 64), oe = __shfl_up(ie, o, 64);
    if (lane >= o) {
      ig += og;
      ie += oe;
    }
  }
  if (lane == 63) {
    scan_g[w] = ig;
    scan_e[w] = ie;
  }
  __syncthreads();
  int n_gt = 0, pg = ig - cg, pe = ie - ce;
#pragma unroll
  for (int i = 0; i < kST / 64; ++i) {
    n_gt += scan_g[i];
    if (i < w) {
      pg += scan_g[i];
      pe += scan_e[i];
    }
  }
  const int need_eq = K - n_gt;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int n = base + i;
    if (key[i] > tau) {
      out[pg++] = n;
    } else if (key[i] == tau) {
      if (pe < need_eq) out[n_gt + pe] = n;
      ++pe;
    }
  }
}

}  // namespace
}  // namespace wptv

using namespace wptv;

namespace {
int64_t score_stride(int N) { return (int64_t)align_up((size_t)N, kKeys); }
}  // namespace

extern "C" int wptv_choice_workspace(int B, int T, int N, size_t* bytes) {
  if (!bytes) return fail(WPTV_E_INVALID, "choice_workspace: bytes is NULL");
  if (B <= 0 || T <= 0 || N <= 0) return fail(WPTV_E_INVALID, "choice_workspace: B=%d T=%d N=%d must be > 0", B, T, N);
  *bytes = (size_t)B * T * score_stride(N) * sizeof(float);
  return WPTV_OK;
}

extern "C" int wptv_exact_choice(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n, int dtype,
                                 const int64_t* positions, const float* lse, int B, int T, int H, int c, int N,
                                 float scale, int top_k, int window, int64_t* chosen, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  if (B <= 0 || T <= 0 || H <= 0 || c <= 0 || N <= 0)
    return fail(WPTV_E_INVALID, "exact_choice: B=%d T=%d H=%d c=%d N=%d must be > 0", B, T, H, c, N);
  if (top_k < 0 || window < 0) return fail(WPTV_E_INVALID, "exact_choice: top_k=%d window=%d", top_k, window);
  const int K = max(0, min(top_k, N - window));
  if (K == 0) return WPTV_OK;
  if (!q || !k || !positions || !lse || !chosen || !workspace)
    return fail(WPTV_E_INVALID, "exact_choice: a required pointer is NULL");
  if (dtype != WPTV_F32 && dtype != WPTV_BF16) return fail(WPTV_E_UNSUPPORTED, "exact_choice: dtype %d", dtype);
  if (H > kMaxRows) return fail(WPTV_E_UNSUPPORTED, "exact_choice: at most %d heads (got %d)", kMaxRows, H);
  if (c > 256) return fail(WPTV_E_UNSUPPORTED, "exact_choice: head width at most 256 (got %d)", c);
  if (!(scale > 0.f)) return fail(WPTV_E_INVALID, "exact_choice: scale must be > 0 (got %g)", (double)scale);
  size_t need = 0;
  wptv_choice_workspace(B, T, N, &need);
  if (workspace_bytes < need)
    return fail(WPTV_E_INVALID, "exact_choice: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  const int64_t ns = score_stride(N);
  const int tb = max(1, min(T, kMaxRows / H));
  const int ntb = (T + tb - 1) / tb;
  const int nkb = (N + kKeys - 1) / kKeys;
  const int64_t grid = (int64_t)B * ntb * nkb;
  if (grid > INT32_MAX || (int64_t)B * T > INT32_MAX) return fail(WPTV_E_INVALID, "exact_choice: grid too large");
  float* scores = static_cast<float*>(workspace);
  const float scale_log2 = scale * kLog2e;
  const bool mfma = dtype == WPTV_BF16 && (c == 64 || c == 128) && aligned(q, 16) && aligned(k, 16) &&
                    k_stride_n % 8 == 0 && k_stride_b % 8 == 0;
  if (mfma && H == 16 && T <= 8) {
    const auto* qq = static_cast<const unsigned short*>(q);
    const auto* kk = static_cast<const unsigned short*>(k);
    const int nkb16 = (N + kH16Rows - 1) / kH16Rows;
    const int grid16 = B * nkb16;
#define WPTV_H16(CC, TT)                                                                                           \
  choice_scores_h16<CC, TT><<<grid16, kST, 0, stream>>>(qq, kk, k_stride_b, k_stride_n, positions, lse, T, N, window, \
                                                        scale_log2, nkb16, scores, ns)
    if (c == 128) {
      if (T <= 1) WPTV_H16(128, 1); else if (T <= 2) WPTV_H16(128, 2); else if (T <= 4) WPTV_H16(128, 4);
      else if (T <= 5) WPTV_H16(128, 5); else WPTV_H16(128, 8);
    } else {
      if (T <= 1) WPTV_H16(64, 1); else if (T <= 2) WPTV_H16(64, 2); else if (T <= 4) WPTV_H16(64, 4);
      else if (T <= 5) WPTV_H16(64, 5); else WPTV_H16(64, 8);
    }
#undef WPTV_H16
  } else if (mfma) {
    const auto* qq = static_cast<const unsigned short*>(q);
    const auto* kk = static_cast<const unsigned short*>(k);
    if (c == 128)
      choice_scores_mfma<128><<<(int)grid, kST, 0, stream>>>(qq, kk, k_stride_b, k_stride_n, positions, lse, T, H, N,
                                                              window, scale_log2, tb, ntb, nkb, scores, ns);
    else
      choice_scores_mfma<64><<<(int)grid, kST, 0, stream>>>(qq, kk, k_stride_b, k_stride_n, positions, lse, T, H, N,
                                                             window, scale_log2, tb, ntb, nkb, scores, ns);
  } else if (dtype == WPTV_BF16) {
    choice_scores_generic<unsigned short><<<(int)grid, kST, 0, stream>>>(
        static_cast<const unsigned short*>(q), static_cast<const unsigned short*>(k), k_stride_b, k_stride_n,
        positions, lse, T, H, c, N, window, scale_log2, tb, ntb, nkb, scores, ns);
  } else {
    choice_scores_generic<float><<<(int)grid, kST, 0, stream>>>(static_cast<const float*>(q),
                                                               static_cast<const float*>(k), k_stride_b, k_stride_n,
                                                               positions, lse, T, H, c, N, window, scale_log2, tb,
                                                               ntb, nkb, scores, ns);
  }
  int status = launched("choice_scores");
  if (status != WPTV_OK) return status;
  // the candidates of a query are at most N rows: in registers up to 8192
  if (N <= kST * 4)
    choice_select_regs<4><<<B * T, kST, 0, stream>>>(scores, ns, positions, N, window, K, chosen);
  else if (N <= kST * 8)
    choice_select_regs<8><<<B * T, kST, 0, stream>>>(scores, ns, positions, N, window, K, chosen);
  else if (N <= kST * 16)
    choice_select_regs<16><<<B * T, kST, 0, stream>>>(scores, ns, positions, N, window, K, chosen);
  else if (N <= kST * 32)
    choice_select_regs<32><<<B * T, kST, 0, stream>>>(scores, ns, positions, N, window, K, chosen);
  else
    choice_select<<<B * T, kST, 0, stream>>>(scores, ns, positions, N, window, K, chosen);
  return launched("choice_select");
}
