// The acceptance step of speculative decoding for gfx950: the reference's
// sampling distribution (Writer._probabilities,
// packages/wpt-inference/src/wpt_inference/__init__.py:173-179) and its
// per-row keep / reject / resample loop (Writer._speculate, :210-229), fused
// over the vocabulary for every row at once, with the draws read from a tape.
//
//   accept_stats   one workgroup per (batch row, position), the single pass
//                  over the vocabulary: the row of scores divided by the
//                  temperature, the top-k threshold (radix select of the k-th
//                  largest, ties kept), the maximum and the softmax
//                  denominator, for a draft position the decision
//                  u * q[draft] < p[draft] and the replacement drawn should it
//                  be the first rejection, argmax_v (max(0, p_v - q_v) / S) / e_v,
//                  and after the last draft the bonus argmax_v p_v / e_v (one
//                  draw from a distribution by the exponential race torch's
//                  multinomial uses); in greedy mode the first maximal index
//                  instead, the draft kept iff it is that index
//   accept_pick    one thread per batch row: the first rejected draft and the
//                  row's tokens from the per-position results
//   tree_walk      greedy verification of a draft tree from the per-node argmax
//
// Each vocabulary row is read once per pass from HBM with coalesced loads and
// kept in registers (ITEMS values per thread); reductions are wavefront
// shuffles, then one LDS step across the 16 wavefronts.
#include "wptv_common.h"

#include <climits>

namespace wptv {
namespace {

constexpr int kT = 1024;       // threads per workgroup
constexpr int kW = kT / 64;    // wavefronts per workgroup
constexpr float kNegInfS = -__builtin_inff();

struct Stats {  // per (batch row, position); arrays of B * P in the workspace
  float* m;     // maximum of scores / temperature over the kept entries
  float* z;     // softmax denominator: sum of exp(s - m) over the kept entries
  float* thr;   // top-k threshold (entries below it have p = 0), -inf without a cut
  int* best;    // first maximal index of the scores
  int* keep;    // 1 if the draft at this position is kept
  int* cand;    // the token drawn if this position is the first rejection (the bonus at the last), -1: none
};

__device__ __forceinline__ float block_max(float x, float* red) {
  x = wave_max(x);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kW; ++w) r = fmaxf(r, red[w]);
  return r;
}

// Sum in a fixed order (wave tree, then wavefronts in index order).
__device__ __forceinline__ float block_sum(float x, float* red) {
  x = wave_sum(x);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = x;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int w = 0; w < kW; ++w) r += red[w];
  return r;
}

// The larger value, the lower index on a tie (torch.argmax's first maximum).
__device__ __forceinline__ void arg_better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i) || (v != v && v2 == v2)) {
    v = v2;
    i = i2;
  }
}

__device__ __forceinline__ int block_argmax(float v, int i, float* redv, int* redi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    arg_better(v, i, v2, i2);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) {
    redv[wave] = v;
    redi[wave] = i;
  }
  __syncthreads();
  float bv = redv[0];
  int bi = redi[0];
  for (int w = 1; w < kW; ++w) arg_better(bv, bi, redv[w], redi[w]);
  return bi;
}

// A row of V floats as a buffer: a load at index v reads row[v], and 0 for
// v >= V (the buffer's range check), from a 32-bit offset per item rather
// than a 64-bit address.
template <typename S>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_resource(const S* row, int V) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<S*>(row), 0, V * (int)sizeof(S), 0x00020000);
}

__device__ __forceinline__ float row_load(__amdgpu_buffer_rsrc_t r, int v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, v * 4, 0, 0));
}

// A scores row of FP32 or bf16 values (the model's logits as they come),
// read as FP32: a bf16 value converts exactly.
template <typename S>
__device__ __forceinline__ float score_load(__amdgpu_buffer_rsrc_t r, int v) {
  if constexpr (sizeof(S) == 2)
    return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, v * 2, 0, 0));
  else
    return row_load(r, v);
}

// x / d, correctly rounded, given y = 1 / d correctly rounded (a uniform
// divisor's reciprocal, computed once): q = x y, then one FMA correction with
// the exact residual x - q d (Markstein's theorem: the result is the rounded
// quotient).  The residual loses bits where it falls below the normal range,
// and the product can overflow: there, and for x = 0's sign, the IEEE division.
// Checked against the division on the CPU: every finite bf16 value and 2e6
// random FP32 values a divisor, at 212 divisors in [0.05, 4.05], no mismatch
// for |x| >= 2^-100 with a finite quotient.
__device__ __forceinline__ float div_by(float x, float d, float y) {
  const float q0 = x * y;
  const float r = fmaf(-q0, d, x);
  const float q = fmaf(r, y, q0);
  return (fabsf(x) >= 0x1p-100f && fabsf(q) < 0x1p+126f) ? q : x / d;
}

// The k-th largest order key among the entries that count (valid[i] and
// key[i] >= floor): a radix select, most significant byte first.
template <int N>
__device__ uint32_t kth_key(const uint32_t (&key)[N], const bool (&valid)[N], uint32_t floor, int k, int* hist,
                            int* sel) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  const int tid = threadIdx.x, lane = tid & 63;
  for (int shift = 24; shift >= 0; shift -= 8) {
    __syncthreads();
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (valid[i] && key[i] >= floor && (key[i] & mask) == prefix) atomicAdd(&hist[(key[i] >> shift) & 255], 1);
    __syncthreads();
    if (tid < 64) {
      // lane l holds bins 4l .. 4l + 3; above[l] = entries in bins >= 4l + 4
      int c[4], total = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) total += (c[e] = hist[4 * lane + e]);
      int suffix = total;  // inclusive suffix sum over lanes >= l
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int other = __shfl_down(suffix, o, 64);
        if (lane + o < 64) suffix += other;
      }
      const uint64_t hit = __builtin_amdgcn_ballot_w64(suffix >= remaining);
      const int top = 63 - __builtin_clzll(hit);  // the highest lane still reaching the k-th entry
      if (lane == top) {
        int above = suffix - total;
        int digit = 4 * lane;
        for (int e = 3; e >= 0; --e) {
          if (above + c[e] >= remaining) {
            digit = 4 * lane + e;
            break;
          }
          above += c[e];
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
  return prefix;
}

// The k-th largest of the valid values (v < V), 0 < k < V.  For k up to the
// number of threads, a floor first: the k-th largest of the threads' own
// maxima.  The k largest maxima are k distinct entries at or above it, so
// the k-th largest entry is too, and the full select then counts only the
// entries at or above the floor (about k of them instead of V, which keeps
// the histogram's atomics off the few bins that hold most of a row).
template <int ITEMS>
__device__ float kth_largest(const float (&s)[ITEMS], int V, int k, int* hist, int* sel) {
  const int tid = threadIdx.x;
  uint32_t key[ITEMS];
  bool valid[ITEMS];
  uint32_t own = 0;
  bool any = false;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    key[i] = order_key(s[i]);
    valid[i] = tid + i * kT < V;
    if (valid[i]) own = max(own, key[i]);
    any |= valid[i];
  }
  uint32_t floor = 0;
  if (k <= kT) {
    const uint32_t mine[1] = {own};
    const bool counts[1] = {any};
    floor = kth_key<1>(mine, counts, 0u, k, hist, sel);
  }
  return key_value(kth_key<ITEMS>(key, valid, floor, k, hist, sel));
}

template <int ITEMS, typename S>
__global__ __launch_bounds__(kT) void accept_stats(const S* __restrict__ scores, int64_t sb, int64_t st,
                                                   const int32_t* __restrict__ firsts, const float* q,
                                                   int64_t qb, int64_t qt, const int64_t* __restrict__ drafts,
                                                   int64_t db, const int32_t* __restrict__ lengths,
                                                   const float* __restrict__ u, const float* e,
                                                   float temperature, int top_k, int greedy, int L, int V,
                                                   Stats stats) {
  __shared__ float redv[kW];
  __shared__ int redi[kW];
  __shared__ int hist[256];
  __shared__ int sel[2];
  const int j = blockIdx.x, b = blockIdx.y, P = L + 1;
  const int n = lengths ? min(max(lengths[b], 0), L) : L;
  if (j > n) return;
  const int64_t first = firsts ? firsts[b] : 0;
  const S* row = scores + b * sb + (first + j) * st;
  const int tid = threadIdx.x;
  // every load of a row issued before the first use; indices past the row
  // read 0, masked after
  const bool draft_pos = j < n;
  const float* qrow = (!greedy && draft_pos) ? q + b * qb + j * qt : nullptr;
  const float* erow = greedy ? nullptr : e + (int64_t)b * V;
  float x[ITEMS];
  const auto rs = row_resource(row, V);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = score_load<S>(rs, tid + i * kT);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = tid + i * kT < V ? x[i] : kNegInfS;
  const int idx = b * P + j;
  if (greedy) {
    // first maximal index of the raw scores (only greedy decisions read it)
    float bv = kNegInfS;
    int bi = INT_MAX;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (tid + i * kT < V) arg_better(bv, bi, x[i], tid + i * kT);
    const int best = block_argmax(bv, bi, redv, redi);
    if (tid == 0) {
      stats.best[idx] = best;
      stats.keep[idx] = (j < n && drafts) ? (drafts[b * db + j] == best) : 0;
    }
    return;
  }
  const float tinv = 1.f / temperature;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = div_by(x[i], temperature, tinv);
  float thr = kNegInfS;
  if (top_k > 0 && top_k < V) thr = kth_largest<ITEMS>(x, V, top_k, hist, sel);
  float mx = kNegInfS;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) mx = fmaxf(mx, x[i]);
  const float m = block_max(mx, redv);
  // exp(s - m) of the kept entries, 0 elsewhere, kept in x for p
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    x[i] = tid + i * kT < V && x[i] >= thr ? expf(x[i] - m) : 0.f;
    part += x[i];
  }
  const float z = block_sum(part, redv);
  // The draw if this position is the first rejected draft: the residual
  // max(0, p - q) normalized by its sum, by the exponential race; at the
  // position after the last draft the bonus draw from p itself (the
  // reference's multinomial of __init__.py:222-229, as argmax_v w_v / e_v).
  // The draft row and then the exponentials are read one at a time, so that
  // no more than two rows are held in registers.
  const float zinv = 1.f / z;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = x[i] * zinv;
  float rest_sum = 1.f;  // the residual's mass (1: the bonus draw from p itself)
  if (draft_pos) {
    float qv[ITEMS];
    const auto rq = row_resource(qrow, V);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) qv[i] = row_load(rq, tid + i * kT);
    float rest = 0.f;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      x[i] = tid + i * kT < V ? fmaxf(x[i] - qv[i], 0.f) : 0.f;
      rest += x[i];
    }
    rest_sum = block_sum(rest, redv);
  }
  float ev[ITEMS];
  const auto re = row_resource(erow, V);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) ev[i] = row_load(re, tid + i * kT);
  float cv = kNegInfS;
  int ci = INT_MAX;
  const float rinv = 1.f / rest_sum;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int v = tid + i * kT;
    if (v < V) arg_better(cv, ci, (draft_pos ? div_by(x[i], rest_sum, rinv) : x[i]) / ev[i], v);
  }
  const int drawn = block_argmax(cv, ci, redv, redi);
  if (tid == 0) {
    stats.m[idx] = m;
    stats.z[idx] = z;
    stats.thr[idx] = thr;
    stats.best[idx] = -1;  // the raw argmax: greedy decisions only
    // a residual with no mass has no draw (the reference's multinomial raises)
    stats.cand[idx] = (!(draft_pos && !(rest_sum > 0.f)) && drawn >= 0 && drawn < V) ? drawn : -1;
    int keep = 0;
    if (j < n) {
      const int64_t d = drafts[b * db + j];
      if (d >= 0 && d < V) {
        const float sd = load_f32(row + d) / temperature;
        const float pd = sd >= thr ? expf(sd - m) * (1.f / z) : 0.f;
        keep = u[(int64_t)b * L + j] * q[b * qb + j * qt + d] < pd;
      }
    }
    stats.keep[idx] = keep;
  }
}

// Each row's tokens from the per-position decisions: the drafts up to the
// first rejected one, then that position's draw (the argmax in greedy mode),
// or every draft and the bonus draw (__init__.py:210-229).  One thread per row.
__global__ __launch_bounds__(64) void accept_pick(const int64_t* __restrict__ drafts, int64_t db,
                                                  const int32_t* __restrict__ lengths, int greedy, int L, int B,
                                                  Stats stats, int64_t* __restrict__ tokens,
                                                  int32_t* __restrict__ n_tokens) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int P = L + 1;
  const int n = lengths ? min(max(lengths[b], 0), L) : L;
  int js = n;  // the first rejected draft, n when every draft is kept (independent loads, not a chain)
  for (int t = n - 1; t >= 0; --t)
    if (!stats.keep[b * P + t]) js = t;
  for (int t = 0; t < P; ++t) tokens[(int64_t)b * P + t] = t < js ? drafts[b * db + t] : -1;
  const int drawn = greedy ? stats.best[b * P + js] : stats.cand[b * P + js];
  tokens[(int64_t)b * P + js] = drawn;
  n_tokens[b] = drawn >= 0 ? js + 1 : -1;
}

// Greedy walk down a draft tree: node i's parent parents[i] < i, the root 0.
__global__ void tree_walk(const int64_t* __restrict__ node_tokens, const int32_t* __restrict__ parents, int B, int M,
                          Stats stats, int64_t* __restrict__ path, int64_t* __restrict__ tokens,
                          int32_t* __restrict__ n_tokens) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int64_t* nt = node_tokens + (int64_t)b * M;
  int64_t* pa = path + (int64_t)b * (M + 1);
  int64_t* tk = tokens + (int64_t)b * (M + 1);
  for (int i = 0; i <= M; ++i) pa[i] = tk[i] = -1;
  int node = 0, depth = 0;
  pa[0] = 0;
  while (true) {
    const int target = stats.best[b * M + node];
    int next = -1;
    for (int c = node + 1; c < M; ++c)
      if (parents[c] == node && nt[c] == target) {
        next = c;
        break;
      }
    if (next < 0) {
      tk[depth] = target;
      break;
    }
    node = next;
    tk[depth] = nt[node];
    ++depth;
    pa[depth] = node;
  }
  n_tokens[b] = depth + 1;
}

Stats carve(void* workspace, int B, int P) {
  char* p = static_cast<char*>(workspace);
  const size_t n = align_up((size_t)B * P * 4, 256);
  Stats s;
  s.m = reinterpret_cast<float*>(p);
  s.z = reinterpret_cast<float*>(p + n);
  s.thr = reinterpret_cast<float*>(p + 2 * n);
  s.best = reinterpret_cast<int*>(p + 3 * n);
  s.keep = reinterpret_cast<int*>(p + 4 * n);
  s.cand = reinterpret_cast<int*>(p + 5 * n);
  return s;
}

size_t stats_bytes(int B, int P) { return 6 * align_up((size_t)B * P * 4, 256); }

int items_for(int V) {
  const int per = (V + kT - 1) / kT;
  if (per <= 4) return 4;
  if (per <= 8) return 8;
  if (per <= 16) return 16;
  if (per <= 32) return 32;
  if (per <= 64) return 64;
  return 0;
}

#define WPTV_ITEMS(V, CALL)                     \
  switch (items_for(V)) {                       \
    case 4: CALL(4); break;                     \
    case 8: CALL(8); break;                     \
    case 16: CALL(16); break;                   \
    case 32: CALL(32); break;                   \
    default: CALL(64); break;                   \
  }

template <typename S>
void launch_stats(dim3 grid, hipStream_t stream, const void* scores, int64_t sb, int64_t st, const int32_t* firsts,
                  const float* q, int64_t qb, int64_t qt, const int64_t* drafts, int64_t db, const int32_t* lengths,
                  const float* u, const float* e, float temperature, int top_k, int greedy, int L, int V, Stats s) {
  const S* rows = static_cast<const S*>(scores);
#define WPTV_STATS(I)                                                                                             \
  hipLaunchKernelGGL((accept_stats<I, S>), grid, dim3(kT), 0, stream, rows, sb, st, firsts, q, qb, qt, drafts, db, \
                     lengths, u, e, temperature, top_k, greedy, L, V, s)
  WPTV_ITEMS(V, WPTV_STATS)
#undef WPTV_STATS
}

}  // namespace
}  // namespace wptv

using namespace wptv;

extern "C" int wptv_accept_workspace(int B, int L, size_t* bytes) {
  if (!bytes) return fail(WPTV_E_INVALID, "accept_workspace: null output pointer");
  if (B <= 0 || L < 0) return fail(WPTV_E_INVALID, "accept_workspace: B must be positive and L >= 0 (got %d, %d)", B, L);
  *bytes = stats_bytes(B, L + 1);
  return WPTV_OK;
}

extern "C" int wptv_accept(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                           const int32_t* firsts, const float* q, int64_t q_stride_b, int64_t q_stride_t,
                           const int64_t* drafts, int64_t drafts_stride_b, const int32_t* lengths, const float* u,
                           const float* e, float temperature, int top_k, int greedy, int B, int L, int V,
                           int64_t* tokens, int32_t* n_tokens, void* workspace, size_t workspace_bytes,
                           hipStream_t stream) {
  if (!scores || !tokens || !n_tokens || (L > 0 && !drafts))
    return fail(WPTV_E_INVALID, "accept: scores, tokens, n_tokens (and drafts when L > 0) must be given");
  if (!greedy && (!e || (L > 0 && (!q || !u))))
    return fail(WPTV_E_INVALID, "accept: sampling needs q, u and e");
  if (B <= 0 || L < 0 || V <= 0)
    return fail(WPTV_E_INVALID, "accept: bad shape B=%d L=%d V=%d", B, L, V);
  if (!greedy && !(temperature > 0.f))
    return fail(WPTV_E_INVALID, "accept: temperature must be positive (got %g)", (double)temperature);
  if (items_for(V) == 0) return fail(WPTV_E_UNSUPPORTED, "accept: a vocabulary of %d is above %d", V, 64 * kT);
  if (scores_dtype != WPTV_F32 && scores_dtype != WPTV_BF16)
    return fail(WPTV_E_UNSUPPORTED, "accept: scores dtype %d is neither fp32 nor bf16", scores_dtype);
  if (!workspace || workspace_bytes < stats_bytes(B, L + 1))
    return fail(WPTV_E_INVALID, "accept: workspace of %zu bytes, %zu needed", workspace_bytes, stats_bytes(B, L + 1));
  const Stats s = carve(workspace, B, L + 1);
  (scores_dtype == WPTV_BF16 ? launch_stats<unsigned short> : launch_stats<float>)(
      dim3(L + 1, B), stream, scores, scores_stride_b, scores_stride_t, firsts, q, q_stride_b, q_stride_t, drafts,
      drafts_stride_b, lengths, u, e, temperature, top_k, greedy, L, V, s);
  int st = launched("accept_stats");
  if (st != WPTV_OK) return st;
  hipLaunchKernelGGL(accept_pick, dim3((B + 63) / 64), dim3(64), 0, stream, drafts, drafts_stride_b, lengths, greedy, L,
                     B, s, tokens, n_tokens);
  return launched("accept_pick");
}

extern "C" int wptv_greedy_tree(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t,
                                int scores_dtype, const int64_t* node_tokens, const int32_t* parents, int B, int M, int V,
                                int64_t* path, int64_t* tokens, int32_t* n_tokens, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  if (!scores || !node_tokens || !parents || !path || !tokens || !n_tokens)
    return fail(WPTV_E_INVALID, "greedy_tree: every pointer must be given");
  if (B <= 0 || M <= 0 || V <= 0) return fail(WPTV_E_INVALID, "greedy_tree: bad shape B=%d M=%d V=%d", B, M, V);
  if (items_for(V) == 0) return fail(WPTV_E_UNSUPPORTED, "greedy_tree: a vocabulary of %d is above %d", V, 64 * kT);
  if (scores_dtype != WPTV_F32 && scores_dtype != WPTV_BF16)
    return fail(WPTV_E_UNSUPPORTED, "greedy_tree: scores dtype %d is neither fp32 nor bf16", scores_dtype);
  if (!workspace || workspace_bytes < stats_bytes(B, M))
    return fail(WPTV_E_INVALID, "greedy_tree: workspace of %zu bytes, %zu needed", workspace_bytes,
                stats_bytes(B, M));
  const Stats s = carve(workspace, B, M);
  // per-node argmax: the stats pass in greedy mode over M positions with no drafts to judge
  (scores_dtype == WPTV_BF16 ? launch_stats<unsigned short> : launch_stats<float>)(
      dim3(M, B), stream, scores, scores_stride_b, scores_stride_t, nullptr, nullptr, 0, 0, nullptr, 0, nullptr,
      nullptr, nullptr, 1.f, 0, 1, M - 1, V, s);
  int st = launched("accept_stats");
  if (st != WPTV_OK) return st;
  hipLaunchKernelGGL(tree_walk, dim3((B + 63) / 64), dim3(64), 0, stream, node_tokens, parents, B, M, s, path, tokens,
                     n_tokens);
  return launched("tree_walk");
}
