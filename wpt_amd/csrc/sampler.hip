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
// Or with the draws the reference's loop makes from a torch generator on the
// device, in its order (wptv_accept_in_order): accept_stats leaves each
// position's p and q of its draft and its residual mass; order_draw replays
// the loop's uniforms (Philox4x32-10, as torch's device generator draws
// them) to find each row's first rejection and the generator offset of its
// multinomial, then draws that multinomial's exponentials over a slice of
// the vocabulary; the last slice of a row to finish joins the row's slices
// and makes its pick.
//
// Each vocabulary row is read once per pass from HBM with coalesced loads and
// kept in registers (ITEMS values per thread); reductions are wavefront
// shuffles, then one LDS step across the 16 wavefronts.
#include "wptv_common.h"

#include <algorithm>
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
  float* pd;    // in-order draws: p of the draft at this position
  float* qd;    // and its q
  float* rest;  // the residual's mass max(0, p - q) summed (1 after the last draft)
  int* arrivals;  // in-order draws: per row, the vocabulary slices whose draws are done (zeroed by accept_stats)
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

// The draws' race: the larger value, the lower index on a tie; a NaN never
// wins (a distribution of NaN has nothing to draw, as torch.multinomial
// refuses it).
__device__ __forceinline__ void arg_better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i) || (v != v && v2 == v2)) {
    v = v2;
    i = i2;
  }
}

// Greedy decisions, torch.argmax's order: a NaN above every number, then the
// larger value; the lower index among equals (NaNs included).
__device__ __forceinline__ void argmax_better(float& v, int& i, float v2, int i2) {
  const bool nan = v != v, nan2 = v2 != v2;
  if (nan2 ? (!nan || i2 < i) : (!nan && (v2 > v || (v2 == v && i2 < i)))) {
    v = v2;
    i = i2;
  }
}

template <bool GREEDY = false>
__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if constexpr (GREEDY)
    argmax_better(v, i, v2, i2);
  else
    arg_better(v, i, v2, i2);
}

template <bool GREEDY = false>
__device__ __forceinline__ int block_argmax(float v, int i, float* redv, int* redi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    better<GREEDY>(v, i, v2, i2);
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
  for (int w = 1; w < kW; ++w) better<GREEDY>(bv, bi, redv[w], redi[w]);
  return bi;
}

// Item i of a thread: entry v = threadIdx.x + i * kT of a row of V values,
// 0 for v >= V.  Each item loads through a buffer over entries i * kT .. V - 1
// (its range check giving the 0s), at the thread's byte offset, the same
// register for every item: no per-item addresses are held.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t item_resource(const T* row, int V, int i) {
  const int start = i * kT;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(row) + start, 0, max(V - start, 0) * (int)sizeof(T),
                                           0x00020000);
}

__device__ __forceinline__ float row_item(const float* row, int V, int i) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_raw_buffer_load_b32(item_resource(row, V, i), threadIdx.x * 4, 0, 0));
}

// A scores row of FP32 or bf16 values (the model's logits as they come):
// the entry's bits as loaded, and their FP32 value (a bf16 value converts
// exactly).  Kept apart so that loads issued after the row's need not wait
// for it.
template <typename S>
__device__ __forceinline__ S score_bits(const S* row, int V, int i) {
  if constexpr (sizeof(S) == 2)
    return __builtin_amdgcn_raw_buffer_load_b16(item_resource(row, V, i), threadIdx.x * 2, 0, 0);
  else
    return row_item(row, V, i);
}

template <typename S>
__device__ __forceinline__ float score_value(S bits) {
  if constexpr (sizeof(S) == 2)
    return bf16_to_f32(bits);
  else
    return bits;
}

// x / d, correctly rounded, given y = 1 / d correctly rounded (a uniform
// divisor's reciprocal, computed once): q = x y, then one FMA correction with
// the exact residual x - q d (Markstein's theorem: the result is the rounded
// quotient).  The residual loses bits where it falls below the normal range,
// and the product can overflow: quot_exact says where the result is the
// rounded quotient, x = 0 or |x| >= 2^-100 with |q| < 2^126.  Checked
// against the division on the CPU: every finite bf16 value and 2e6 random
// FP32 values a divisor at 212 divisors in [0.05, 4.05], and 2e9 random
// (x, d) pairs with d over 2^-60 .. 2^60: no mismatch where it holds.
__device__ __forceinline__ float quot(float x, float d, float y) {
  const float q0 = x * y;
  return fmaf(fmaf(-q0, d, x), y, q0);
}

__device__ __forceinline__ bool quot_exact(float x, float q) {
  return (x == 0.f) | ((fabsf(x) >= 0x1p-100f) & (fabsf(q) < 0x1p+126f));  // no branches
}

// x / d correctly rounded: the fast quotient, and the IEEE division only in
// a wavefront where some lane needs it (a branch every lane takes alike; the
// empty volatile statement keeps the compiler from computing the division
// everywhere and selecting).
__device__ __forceinline__ float div_by(float x, float d, float y) {
  float q = quot(x, d, y);
  const bool exact = quot_exact(x, q);
  if (__builtin_amdgcn_ballot_w64(!exact)) {
    asm volatile("");
    if (!exact) q = x / d;
  }
  return q;
}

// e^t for t <= 0 (NaN gives 0): 2^(t log2 e) with the product carried in two
// parts (its rounding error by an FMA, plus t times the low part of log2 e:
// a Cody-Waite style split of the constant, Cody and Waite, "Software Manual
// for the Elementary Functions", 1980), split at its nearest integer n, the
// fraction's power on the hardware's exp2 and scaled by 2^n; below ln 2^-149
// the result is 0.  A non-positive argument needs no overflow branch.
// Contraction off: ph - n must subtract the rounded product, whose rounding
// error pl carries.
__device__ __forceinline__ float exp_nonpos(float t) {
#pragma clang fp contract(off)
  const float ph = t * kLog2e;
  const float pl = fmaf(t, 0x1.4ae0bep-26f, fmaf(t, kLog2e, -ph));
  const float n = __builtin_rintf(ph);
  const float r = __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), (int)n);
  return t >= -0x1.9d1da0p+6f ? r : 0.f;
}

// The k-th largest order key among the entries that count (key_at(i, key)
// true and key >= floor): a radix select, most significant byte first.  The
// keys are formed in each pass rather than held, which keeps N registers free.
template <int N, typename KeyAt>
__device__ uint32_t kth_key(KeyAt key_at, uint32_t floor, int k, int* hist, int* sel) {
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  const int tid = threadIdx.x, lane = tid & 63;
  for (int shift = 24; shift >= 0; shift -= 8) {
    __syncthreads();
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
      uint32_t key;
      if (key_at(i, key) && key >= floor && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
    }
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

// The k-th largest of a row's V values, 0 < k < V, the entries past the row
// (v >= V) holding -inf: they are below or equal to every entry, so with
// k < V they do not move the k-th largest and are counted like the others.
// For k up to the number of threads, a floor first: the k-th largest of the
// threads' own maxima.  The k largest maxima are k distinct entries at or
// above it, so the k-th largest entry is too, and the full select then
// counts only the entries at or above the floor (about k of them instead of
// V, which keeps the histogram's atomics off the few bins that hold most of
// a row).
// With a floor, each thread first gathers its entries at or above it (two
// slots): the radix passes then read those instead of every entry, unless a
// thread holds more than two (then they read every entry, as without one).
template <int ITEMS>
__device__ float kth_largest(const float (&s)[ITEMS], int k, int* hist, int* sel, float* red) {
  const auto entry = [&](int i, uint32_t& key) {
    key = order_key(s[i]);
    return true;
  };
  uint32_t own = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) own = max(own, order_key(s[i]));
  if (k > kT) return key_value(kth_key<ITEMS>(entry, 0u, k, hist, sel));
  const uint32_t floor = kth_key<1>(
      [&](int, uint32_t& key) {
        key = own;
        return true;
      },
      0u, k, hist, sel);
  uint32_t c0 = 0, c1 = 0;
  int count = 0;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const uint32_t key = order_key(s[i]);
    const bool at = key >= floor;
    c1 = at && count == 1 ? key : c1;
    c0 = at && count == 0 ? key : c0;
    count += at;
  }
  if (block_max((float)count, red) <= 2.f)
    return key_value(kth_key<2>(
        [&](int i, uint32_t& key) {
          key = i ? c1 : c0;
          return i < count;
        },
        floor, k, hist, sel));
  return key_value(kth_key<ITEMS>(entry, floor, k, hist, sel));
}

// QLDS: the draft row is copied into LDS by DMA and the exponentials loaded
// into registers at the start (after the top-k select when CUT, whose passes
// need the registers), so that the rows stream in together, and the draft's
// own p and q come from the thread that holds its score; needs the row in
// LDS (V <= 32768, a multiple of 4 floats, 16-byte aligned).  CUT: a top-k
// cut (0 < top_k < V).  ORDER: no tape; the position's p and q of its draft
// and its residual mass are left for order_draw, which makes the draws.
template <int ITEMS, typename S, bool QLDS, bool CUT, bool ORDER>
__global__ __launch_bounds__(kT) void accept_stats(const S* __restrict__ scores, int64_t sb, int64_t st,
                                                   const int32_t* __restrict__ firsts, const float* q,
                                                   int64_t qb, int64_t qt, const int64_t* __restrict__ drafts,
                                                   int64_t db, const int32_t* __restrict__ lengths,
                                                   const float* __restrict__ u, const float* e,
                                                   float temperature, int top_k, int greedy, int B, int L,
                                                   int V, Stats stats) {
  __shared__ float redv[kW];
  __shared__ int redi[kW];
  __shared__ int hist[256];
  __shared__ int sel[2];
  __shared__ __attribute__((aligned(16))) float qs[QLDS ? ITEMS * kT : 1];  // QLDS: the draft row, qs[v] = q[v]
  // A row's P positions on one XCD (workgroups are dealt to the 8 XCDs in
  // turn, so those whose index agrees mod 8 share one): its exponentials row
  // is read from HBM once and found in that XCD's L2 by the others.
  const int P = L + 1, slot = blockIdx.x >> 3;
  const int b = 8 * (slot / P) + (blockIdx.x & 7), j = slot % P;
  if constexpr (ORDER) {  // order_draw, the next launch, counts each row's slices from zero
    if (blockIdx.x == 0)
      for (int i = threadIdx.x; i < B; i += kT) stats.arrivals[i] = 0;
  }
  if (b >= B) return;
  const int n = lengths ? min(max(lengths[b], 0), L) : L;
  if (j > n) return;
  const int64_t first = firsts ? firsts[b] : 0;
  const S* row = scores + b * sb + (first + j) * st;
  const int tid = threadIdx.x;
  // every load of a row issued before the first use; indices past the row
  // read 0, masked after
  const bool draft_pos = j < n;
  const float* qrow = (!greedy && draft_pos) ? q + b * qb + j * qt : nullptr;
  const float* erow = (greedy || ORDER) ? nullptr : e + (int64_t)b * V;
  S bits[ITEMS];
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) bits[i] = score_bits<S>(row, V, i);
  const int idx = b * P + j;
  float x[ITEMS];
  if (greedy) {
    // first maximal index of the raw scores (only greedy decisions read it)
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) x[i] = tid + i * kT < V ? score_value<S>(bits[i]) : kNegInfS;
    float bv = kNegInfS;
    int bi = INT_MAX;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (tid + i * kT < V) argmax_better(bv, bi, x[i], tid + i * kT);
    const int found = block_argmax<true>(bv, bi, redv, redi);
    const int best = found >= 0 && found < V ? found : -1;
    if (tid == 0) {
      stats.best[idx] = best;
      stats.keep[idx] = (j < n && drafts && best >= 0) ? (drafts[b * db + j] == best) : 0;
    }
    return;
  }
  const int64_t d = draft_pos ? drafts[b * db + j] : -1;
  float ev[ITEMS];
  if constexpr (QLDS) {
    // the exponentials, then the draft row by DMA (last: the first wait for
    // it is before the residual): wave w's instruction c moves floats 4096 c
    // + 256 w .. + 255 to the same entries of qs (16 bytes a lane); the range
    // check covers the row's V * 4 bytes
    if constexpr (!CUT && !ORDER) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) ev[i] = row_item(erow, V, i);
    }
    if (draft_pos) {
      i32x4 rq = buffer_resource(qrow);
      rq[2] = V * 4;
      const uint32_t lds = lds_address(qs) + 1024u * (uint32_t)__builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
      for (int c = 0; c < ITEMS / 4; ++c) dma_16B(rq, 16u * (uint32_t)(c * kT + tid), lds + 16384u * c);
    }
  }
  // The entries past the row (v >= V) are -inf from here on: each later
  // phase then gives them p = 0, a residual of 0 (the draft row reads 0
  // there) and a race value of 0 / 0, which never wins.
  const float tinv = 1.f / temperature;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = div_by(score_value<S>(bits[i]), temperature, tinv);
  if (V < ITEMS * kT) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (tid + i * kT >= V) x[i] = kNegInfS;
    if constexpr (QLDS) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i)
        if (tid + i * kT >= V) qs[tid + i * kT] = 0.f;  // as the range-checked DMA writes them
    }
  }
  float thr = kNegInfS;
  if constexpr (CUT) {
    thr = kth_largest<ITEMS>(x, top_k, hist, sel, redv);
    if constexpr (QLDS && !ORDER) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) ev[i] = row_item(erow, V, i);
    }
  }
  float mx = kNegInfS;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) mx = fmaxf(mx, x[i]);
  const float m = block_max(mx, redv);
  // exp(s - m) of the kept entries, 0 elsewhere, kept in x for p
  float part = 0.f;
  if constexpr (CUT) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      x[i] = x[i] >= thr ? exp_nonpos(x[i] - m) : 0.f;
      part += x[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      x[i] = exp_nonpos(x[i] - m);
      part += x[i];
    }
  }
  const float z = block_sum(part, redv);
  // The draw if this position is the first rejected draft: the residual
  // max(0, p - q) normalized by its sum, by the exponential race; at the
  // position after the last draft the bonus draw from p itself (the
  // reference's multinomial of __init__.py:222-229, as argmax_v w_v / e_v).
  const float zinv = 1.f / z;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) x[i] = x[i] * zinv;
  // QLDS: p of the draft, held by thread d mod kT as item d / kT
  const bool owner = QLDS && d >= 0 && d < V && (int)(d & (kT - 1)) == tid;
  float pd = 0.f;
  if (owner) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
      if (i == (int)(d >> 10)) pd = x[i];
  }
  float rest_sum = 1.f;  // the residual's mass (1: the bonus draw from p itself)
  if (draft_pos) {
    float rest = 0.f;
    if constexpr (QLDS) {
      wait_vmcnt<0>();  // this wavefront's DMA has landed
      __syncthreads();  // and every other's
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        x[i] = fmaxf(x[i] - qs[tid + i * kT], 0.f);
        rest += x[i];
      }
    } else {
      // the draft row read now, one row in registers at a time
      float qv[ITEMS];
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) qv[i] = row_item(qrow, V, i);
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) {
        x[i] = fmaxf(x[i] - qv[i], 0.f);
        rest += x[i];
      }
    }
    rest_sum = block_sum(rest, redv);
  }
  if constexpr (ORDER) {
    if (tid == 0) {
      stats.m[idx] = m;
      stats.z[idx] = z;
      stats.thr[idx] = thr;
      stats.best[idx] = -1;
      stats.rest[idx] = rest_sum;
      if constexpr (!QLDS) {
        float pdg = 0.f, qdg = 0.f;  // an out-of-range draft is rejected: u * 0 < 0 never holds
        if (d >= 0 && d < V) {
          const float sd = load_f32(row + d) / temperature;
          pdg = sd >= thr ? exp_nonpos(sd - m) * zinv : 0.f;
          qdg = q[b * qb + j * qt + d];
        }
        stats.pd[idx] = pdg;
        stats.qd[idx] = qdg;
      } else if (!(d >= 0 && d < V)) {
        stats.pd[idx] = 0.f;
        stats.qd[idx] = 0.f;
      }
    }
    if (owner) {
      stats.pd[idx] = pd;
      stats.qd[idx] = qs[d];
    }
    return;
  } else {
    if constexpr (!QLDS) {
#pragma unroll
      for (int i = 0; i < ITEMS; ++i) ev[i] = row_item(erow, V, i);
    }
    // each thread's entries in index order: the first of its largest values
    // wins (a NaN never does), as arg_better's order across threads has it
    float cv = kNegInfS;
    int ci = INT_MAX;
    const float rinv = 1.f / rest_sum;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const float c = (draft_pos ? div_by(x[i], rest_sum, rinv) : x[i]) / ev[i];
      if (c > cv) {
        cv = c;
        ci = tid + i * kT;
      }
    }
    const int drawn = block_argmax(cv, ci, redv, redi);
    if (tid == 0) {
      stats.m[idx] = m;
      stats.z[idx] = z;
      stats.thr[idx] = thr;
      stats.best[idx] = -1;  // the raw argmax: greedy decisions only
      // a residual with no mass has no draw (the reference's multinomial raises)
      stats.cand[idx] = (!(draft_pos && !(rest_sum > 0.f)) && drawn >= 0 && drawn < V) ? drawn : -1;
      if constexpr (!QLDS) {
        int keep = 0;
        if (d >= 0 && d < V) {
          const float sd = load_f32(row + d) / temperature;
          const float pdg = sd >= thr ? exp_nonpos(sd - m) * zinv : 0.f;
          keep = u[(int64_t)b * L + j] * q[b * qb + j * qt + d] < pdg;
        }
        stats.keep[idx] = keep;
      } else if (!(d >= 0 && d < V)) {
        stats.keep[idx] = 0;
      }
    }
    // the same p as exp(s_d - m) * (1 / z) of the draft's score: the decision u * q[d] < p[d]
    if (owner) stats.keep[idx] = u[(int64_t)b * L + j] * qs[d] < pd;
  }
}

// ---- the draws of torch's device generator, in the reference's order --------
//
// torch draws on the GPU from Philox4x32-10 (Salmon, Moraes, Dror and Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC 2011) through hipRAND:
// a call that draws numel floats at the generator's offset o runs S threads
// (256 a workgroup, min(multiprocessors x max threads a multiprocessor / 256,
// ceil(numel / 256)) workgroups), and thread t takes block (o / 4 + k) of its
// subsequence t, word w of it giving entry 4 S k + S w + t; each float is
// (word + 1) 2^-32 rounded, in (0, 1]; the call then moves the offset on by
// 4 ceil(numel / 4 S).  The reference's loop draws, row by row, one
// torch.rand(()) per draft it judges (offset + 4 each; a value of 1 read as
// 0) and then one torch.multinomial(w, 1) over the vocabulary, which is
// argmax_v w_v / e_v over numel = V exponentials e_v = -log u_v (u at or
// above 1 - 2^-24 taken as giving 2^-24) and moves the offset by 4 more.

constexpr int kDT = 256;        // threads of a draw workgroup
constexpr int kSlices = 32;     // draw workgroups a row's multinomial is shared over
constexpr int kScanMax = 3072;  // positions B (L + 1) the in-order scan may read (16 B P bytes of LDS)

struct Order {
  const int64_t* state;  // the generator's [seed, offset] on the device
  int64_t* next;         // where the offset after this call's draws is written
  uint32_t threads;      // S of the multinomial's draw (of V entries, or of B V when joint)
  int joint;             // one multinomial over every row's V entries (L = 0: Writer._sample's)
  int64_t joint_step;    // that draw's offset step
  float2* parts;         // per row and slice: the slice's race winner (value, index bits)
};

__device__ __forceinline__ uint32_t philox_word(uint64_t counter, uint64_t subsequence, uint64_t seed, int word) {
  uint32_t c0 = (uint32_t)counter, c1 = (uint32_t)(counter >> 32);
  uint32_t c2 = (uint32_t)subsequence, c3 = (uint32_t)(subsequence >> 32);
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;  // the key schedule's Weyl increments
    k1 += 0xBB67AE85u;
  }
  return word == 0 ? c0 : word == 1 ? c1 : word == 2 ? c2 : c3;
}

__device__ __forceinline__ float word_uniform(uint32_t w) { return 0x1p-32f + (float)w * 0x1p-32f; }

// Entry li of a draw of S threads at offset o.
__device__ __forceinline__ float drawn_uniform(uint64_t seed, uint64_t o, uint32_t li, uint32_t S) {
  const uint32_t block = li / (4u * S), rest = li - block * 4u * S, word = rest / S;
  return word_uniform(philox_word(o / 4 + block, rest - word * S, seed, (int)word));
}

__device__ __forceinline__ float drawn_exponential(float u) {
  return -1.f * (u >= 1.f - 0x1p-24f ? -0x1p-24f : __logf(u));
}

// What a verify step does with a row's count once it is known, in the pick's
// own thread (COMMIT): the cache takes back the rejected drafts (the
// reference's Rows.undo, cache.py:69-77: lengths = before + kept, kept outside
// 0 .. the tokens read taken as the nearest end) and the last written token
// becomes the row's pending token; a row that wrote nothing keeps its pending
// token and raises *failed.
struct Commit {
  int64_t* lengths;
  const int64_t* before;
  int64_t* feeds;
  int64_t feeds_stride;
  int* failed;
  int64_t* written;
};

__device__ inline void commit_row(const Commit& c, int b, int n, int64_t last) {
  const int64_t start = c.before[b], read = c.lengths[b] - start;
  c.lengths[b] = start + min(max((int64_t)n, (int64_t)0), read);
  if (n < 1) {
    if (c.failed) *c.failed = 1;
    return;
  }
  c.feeds[(int64_t)b * c.feeds_stride] = last;
  if (c.written) c.written[b] += n;
}

// The draws of row b's multinomial over vocabulary slice s (blockIdx.x = b
// kSlices + s).  Each workgroup first replays the loop up to its row: the
// uniforms u_t = U(o + 4 t) it may read, every row's drafts' p and q, then
// wavefront 0 takes the rows in turn (lane j judging draft j:
// u * q < p keeps it), a row of n judged drafts moving t on by n + 1.  Row
// b's multinomial then draws at offset o + 4 t from position js's
// distribution: the residual max(0, p - q) over its mass, or p after the
// last draft; its p from the statistics of that position (the same steps as
// accept_stats, so the same bits).  Only entries with w > 0 draw an
// exponential: 0 / e is 0 for every e the draw can give.
//
// The row's pick runs in the last of its slices to finish: each slice stores
// its race winner with a device-scope store, waits for it to complete, then
// counts itself in stats.arrivals[b] (a device-scope atomic, zeroed by
// accept_stats); the slice that counts the row's last reads the kSlices
// winners back with device-scope loads (they see every XCD's stores), joins
// them in index order and writes the row's tokens (the drafts up to the
// first rejected one, then the draw: __init__.py:210-229), its count, and
// with COMMIT its cache length, pending token and running count; the last
// row's pick also writes the generator's next offset.  No workgroup waits
// for another.
template <int N, typename S, bool CUT, bool COMMIT>
__global__ __launch_bounds__(kDT) void order_draw(const S* __restrict__ scores, int64_t sb, int64_t st,
                                                  const int32_t* __restrict__ firsts, const float* __restrict__ q,
                                                  int64_t qb, int64_t qt, const int32_t* __restrict__ lengths,
                                                  float temperature, int B, int L, int V, Stats stats, Order order,
                                                  const int64_t* __restrict__ drafts, int64_t db,
                                                  int64_t* __restrict__ tokens, int32_t* __restrict__ n_tokens,
                                                  Commit commit) {
  // the replay's tables, sized at launch: uniforms B P, drafts' p and q B L each, lengths B
  extern __shared__ __attribute__((aligned(16))) float scan_lds[];
  float* utab = scan_lds;
  float* spd = utab + B * (L + 1);
  float* sqd = spd + B * L;
  int* slen = reinterpret_cast<int*>(sqd + B * L);
  __shared__ float redv[kDT / 64];
  __shared__ int redi[kDT / 64];
  __shared__ int found[2];
  __shared__ int last;
  const int b = blockIdx.x / kSlices, s = blockIdx.x % kSlices, tid = threadIdx.x;
  if (b >= B) return;
  const int P = L + 1;
  const uint64_t seed = (uint64_t)order.state[0], base = (uint64_t)order.state[1];
  int js = 0, t_draw = 0;
  if (!order.joint) {
    const int reach = (b + 1) * P;  // t stays below this up to row b
    for (int t = tid; t < reach; t += kDT) {
      const float u = word_uniform(philox_word(base / 4 + (uint64_t)t, 0, seed, 0));
      utab[t] = u == 1.f ? 0.f : u;
    }
    for (int r = tid; r <= b; r += kDT) slen[r] = lengths ? min(max(lengths[r], 0), L) : L;
    for (int k = tid; k < (b + 1) * L; k += kDT) {
      const int r = k / L, j = k - r * L;
      spd[k] = stats.pd[r * P + j];
      sqd[k] = stats.qd[r * P + j];
    }
    __syncthreads();
    if (tid < 64) {
      int t = 0;
      for (int r = 0; r <= b; ++r) {
        const int len = slen[r];
        const bool rejected = tid < len && !(utab[t + tid] * sqd[r * L + tid] < spd[r * L + tid]);
        const uint64_t mask = __builtin_amdgcn_ballot_w64(rejected);
        const int first = mask ? __builtin_ctzll(mask) : len;
        const int n = first < len ? first + 1 : len;
        if (r == b) {
          js = first;
          t_draw = t + n;
        }
        t += n + 1;
      }
      if (tid == 0) {
        found[0] = js;
        found[1] = t_draw;
      }
    }
    __syncthreads();
    js = found[0];
    t_draw = found[1];
  }
  const int len = order.joint ? 0 : (lengths ? min(max(lengths[b], 0), L) : L);
  const bool draft_pos = js < len;
  const int idx = b * P + js;
  const float m = stats.m[idx], z = stats.z[idx], thr = stats.thr[idx], rest = stats.rest[idx];
  const float zinv = 1.f / z, rinv = 1.f / rest, tinv = 1.f / temperature;
  const int64_t first = firsts ? firsts[b] : 0;
  const S* row = scores + b * sb + (first + js) * st;
  const float* qrow = draft_pos ? q + b * qb + js * qt : nullptr;
  const uint64_t o = base + 4 * (uint64_t)t_draw;
  const uint32_t li0 = order.joint ? (uint32_t)b * (uint32_t)V : 0u;
  const int per = (V + kSlices - 1) / kSlices, v0 = s * per, v1 = min(V, v0 + per);
  // every load first: the slice's scores and draft entries
  S bits[N];
  float qv[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int v = v0 + tid + i * kDT;
    bits[i] = v < v1 ? row[v] : S(0);
    qv[i] = (draft_pos && v < v1) ? qrow[v] : 0.f;
  }
  float cv = kNegInfS;
  int ci = INT_MAX;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int v = v0 + tid + i * kDT;
    if (v >= v1) continue;
    const float x = div_by(score_value<S>(bits[i]), temperature, tinv);
    float w;
    if constexpr (CUT)
      w = x >= thr ? exp_nonpos(x - m) : 0.f;
    else
      w = exp_nonpos(x - m);
    w = w * zinv;
    if (draft_pos) w = div_by(fmaxf(w - qv[i], 0.f), rest, rinv);
    float c = w;  // 0 (and a NaN) as w / e would give them
    if (w > 0.f) c = w / drawn_exponential(drawn_uniform(seed, o, li0 + (uint32_t)v, order.threads));
    if (c > cv) {
      cv = c;
      ci = v;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float v2 = __shfl_xor(cv, off, 64);
    const int i2 = __shfl_xor(ci, off, 64);
    arg_better(cv, ci, v2, i2);
  }
  if ((tid & 63) == 0) {
    redv[tid >> 6] = cv;
    redi[tid >> 6] = ci;
  }
  __syncthreads();
  if (tid == 0) {
    float bv = redv[0];
    int bi = redi[0];
#pragma unroll
    for (int w = 1; w < kDT / 64; ++w) arg_better(bv, bi, redv[w], redi[w]);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(order.parts + b * kSlices + s),
                       __builtin_bit_cast(uint64_t, make_float2(bv, __int_as_float(bi))), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::: "memory");
    wait_vmcnt<0>();
    last = __hip_atomic_fetch_add(stats.arrivals + b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kSlices - 1;
  }
  __syncthreads();
  if (!last || tid >= 64) return;

  // the row's pick: lane l < kSlices holds slice l's winner
  const int lane = tid;
  float bv = kNegInfS;
  int bi = INT_MAX;
  if (lane < kSlices) {
    const float2 part = __builtin_bit_cast(
        float2, __hip_atomic_load(reinterpret_cast<uint64_t*>(order.parts + b * kSlices + lane), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT));
    bv = part.x;
    bi = __float_as_int(part.y);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float v2 = __shfl_xor(bv, off, 64);
    const int i2 = __shfl_xor(bi, off, 64);
    arg_better(bv, bi, v2, i2);
  }
  int pick = bi >= 0 && bi < V ? bi : -1;
  // a residual with no mass has no draw (the reference's multinomial raises)
  if (draft_pos && !(rest > 0.f)) pick = -1;
  for (int t = lane; t < P; t += 64) tokens[(int64_t)b * P + t] = t < js ? drafts[b * db + t] : (t == js ? pick : -1);
  if (lane != 0) return;
  n_tokens[b] = pick >= 0 ? js + 1 : -1;
  if constexpr (COMMIT) commit_row(commit, b, pick >= 0 ? js + 1 : -1, pick);
  if (b == B - 1) *order.next = order.state[1] + (order.joint ? order.joint_step : 4 * ((int64_t)t_draw + 1));
}


// Each row's tokens from the per-position decisions: the drafts up to the
// first rejected one, then that position's draw (the argmax in greedy mode),
// or every draft and the bonus draw (__init__.py:210-229).  One thread per row.
template <bool COMMIT>
__global__ __launch_bounds__(64) void accept_pick(const int64_t* __restrict__ drafts, int64_t db,
                                                  const int32_t* __restrict__ lengths, int greedy, int L, int B,
                                                  Stats stats, int64_t* __restrict__ tokens,
                                                  int32_t* __restrict__ n_tokens, Commit commit) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int P = L + 1;
  const int* drawn_at = greedy ? stats.best : stats.cand;
  constexpr int kMaxP = 16;
  if (P <= kMaxP) {
    // every load of the row at once (one memory round trip), then the choice in registers
    int keep[kMaxP], drawn[kMaxP];
    int64_t draft[kMaxP];
    const int given = lengths ? lengths[b] : L;
    // indices clamped into the row: the loads need no branches; entries past
    // P (or L) are never chosen
#pragma unroll
    for (int t = 0; t < kMaxP; ++t) {
      keep[t] = stats.keep[b * P + min(t, P - 1)];
      drawn[t] = drawn_at[b * P + min(t, P - 1)];
      draft[t] = L > 0 ? drafts[b * db + min(t, L - 1)] : -1;
    }
    const int n = min(max(given, 0), L);
    int js = n;  // the first rejected draft, n when every draft is kept
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
      if (t < n && js == n && !keep[t]) js = t;
    int pick = -1;
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
      if (t == js) pick = drawn[t];
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
      if (t < P) tokens[(int64_t)b * P + t] = t < js ? draft[t] : (t == js ? pick : -1);
    n_tokens[b] = pick >= 0 ? js + 1 : -1;
    if constexpr (COMMIT) commit_row(commit, b, pick >= 0 ? js + 1 : -1, pick);
    return;
  }
  const int n = lengths ? min(max(lengths[b], 0), L) : L;
  int js = n;  // the first rejected draft, n when every draft is kept (independent loads, not a chain)
  for (int t = n - 1; t >= 0; --t)
    if (!stats.keep[b * P + t]) js = t;
  for (int t = 0; t < P; ++t) tokens[(int64_t)b * P + t] = t < js ? drafts[b * db + t] : -1;
  const int pick = drawn_at[b * P + js];
  tokens[(int64_t)b * P + js] = pick;
  n_tokens[b] = pick >= 0 ? js + 1 : -1;
  if constexpr (COMMIT) commit_row(commit, b, pick >= 0 ? js + 1 : -1, pick);
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
  // a given best of -1 ends the walk with nothing written
  n_tokens[b] = tk[depth] >= 0 ? depth + 1 : -1;
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
  s.pd = reinterpret_cast<float*>(p + 6 * n);
  s.qd = reinterpret_cast<float*>(p + 7 * n);
  s.rest = reinterpret_cast<float*>(p + 8 * n);
  s.arrivals = nullptr;
  return s;
}

// The per-position arrays, then the in-order draws' per-row arrival counts and per-slice results.
size_t stats_bytes(int B, int P) { return 9 * align_up((size_t)B * P * 4, 256); }
size_t order_bytes(int B) { return align_up((size_t)B * 8, 256) + align_up((size_t)B * kSlices * 8, 256); }

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

// Greedy decisions alone (no drafts' distributions to form): each (batch
// row, position)'s first maximal index of the raw scores, by one workgroup of
// kGT threads reading the row 16 bytes a lane, every load of a thread issued
// before the first comparison; torch.argmax's order (argmax_better: a NaN
// the largest, then the larger value, then the lower index), so the index does
// not depend on how the row is shared out.  Rows 16-byte aligned, V a
// multiple of 16 / sizeof(S).
constexpr int kGT = 256;
constexpr int kGLoads = 16;  // 16-byte loads a thread has in flight

template <typename S>
__global__ __launch_bounds__(kGT) void greedy_argmax(const S* __restrict__ scores, int64_t sb, int64_t st,
                                                     const int32_t* __restrict__ firsts,
                                                     const int64_t* __restrict__ drafts, int64_t db,
                                                     const int32_t* __restrict__ lengths, int B, int L, int V,
                                                     Stats stats) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int kPer = 16 / (int)sizeof(S);  // values a 16-byte load holds
  __shared__ float redv[kGT / 64];
  __shared__ int redi[kGT / 64];
  const int P = L + 1;
  const int b = blockIdx.x / P, j = blockIdx.x % P;
  if (b >= B) return;
  const int n = lengths ? min(max(lengths[b], 0), L) : L;
  if (j > n) return;
  const int64_t first = firsts ? firsts[b] : 0;
  const u32x4* row = reinterpret_cast<const u32x4*>(scores + b * sb + (first + j) * st);
  const int chunks = V / kPer, tid = threadIdx.x;
  float bv = kNegInfS;
  int bi = INT_MAX;
  for (int c0 = 0; c0 < chunks; c0 += kGT * kGLoads) {
    u32x4 w[kGLoads];
#pragma unroll
    for (int u = 0; u < kGLoads; ++u) {
      const int c = c0 + tid + u * kGT;
      w[u] = c < chunks ? row[c] : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kGLoads; ++u) {
      const int c = c0 + tid + u * kGT;
      if (c >= chunks) continue;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        float x;
        if constexpr (sizeof(S) == 2)
          x = __uint_as_float(e & 1 ? (w[u][e >> 1] & 0xffff0000u) : (w[u][e >> 1] << 16));
        else
          x = __uint_as_float(w[u][e]);
        argmax_better(bv, bi, x, c * kPer + e);
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o, 64);
    const int i2 = __shfl_xor(bi, o, 64);
    argmax_better(bv, bi, v2, i2);
  }
  const int wave = tid >> 6, lane = tid & 63;
  if (lane == 0) {
    redv[wave] = bv;
    redi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = redv[0];
    int i = redi[0];
#pragma unroll
    for (int w = 1; w < kGT / 64; ++w) argmax_better(v, i, redv[w], redi[w]);
    const int idx = b * P + j;
    const int best = i >= 0 && i < V ? i : -1;
    stats.best[idx] = best;
    stats.keep[idx] = (j < n && drafts && best >= 0) ? (drafts[b * db + j] == best) : 0;
  }
}

// One workgroup per (batch row, position): 8 ceil(B / 8) (L + 1) of them,
// those past B returning at once.
template <typename S, bool ORDER = false>
void launch_stats(int B, hipStream_t stream, const void* scores, int64_t sb, int64_t st, const int32_t* firsts,
                  const float* q, int64_t qb, int64_t qt, const int64_t* drafts, int64_t db, const int32_t* lengths,
                  const float* u, const float* e, float temperature, int top_k, int greedy, int L, int V, Stats s) {
  const S* rows = static_cast<const S*>(scores);
  constexpr int kPer = 16 / (int)sizeof(S);
  if (greedy && V % kPer == 0 && sb % kPer == 0 && st % kPer == 0 && aligned(scores, 16)) {
    hipLaunchKernelGGL(greedy_argmax<S>, dim3(B * (L + 1)), dim3(kGT), 0, stream, rows, sb, st, firsts, drafts, db,
                       lengths, B, L, V, s);
    return;
  }
  const dim3 grid(8 * ((B + 7) / 8) * (L + 1));
  // the draft rows through LDS when every row is 16-byte aligned and fits
  const bool qlds = !greedy && q && V <= 32 * kT && V % 4 == 0 && aligned(q, 16) && qb % 4 == 0 && qt % 4 == 0;
  const bool cut = !greedy && top_k > 0 && top_k < V;
#define WPTV_STATS_Q(I, QL, CU)                                                                                  \
  hipLaunchKernelGGL((accept_stats<I, S, QL, CU, ORDER>), grid, dim3(kT), 0, stream, rows, sb, st, firsts, q, qb,  \
                     qt, drafts, db, lengths, u, e, temperature, top_k, greedy, B, L, V, s)
#define WPTV_STATS_C(I, QL)            \
  if (cut) WPTV_STATS_Q(I, QL, true);  \
  else WPTV_STATS_Q(I, QL, false);
#define WPTV_STATS(I)                  \
  if constexpr (I <= 32) {             \
    if (qlds) {                        \
      WPTV_STATS_C(I, true)            \
    } else {                           \
      WPTV_STATS_C(I, false)           \
    }                                  \
  } else {                             \
    WPTV_STATS_C(I, false)             \
  }
  WPTV_ITEMS(V, WPTV_STATS)
#undef WPTV_STATS
#undef WPTV_STATS_C
#undef WPTV_STATS_Q
}

}  // namespace
}  // namespace wptv

using namespace wptv;

extern "C" int wptv_accept_workspace(int B, int L, size_t* bytes) {
  if (!bytes) return fail(WPTV_E_INVALID, "accept_workspace: null output pointer");
  if (B <= 0 || L < 0) return fail(WPTV_E_INVALID, "accept_workspace: B must be positive and L >= 0 (got %d, %d)", B, L);
  *bytes = stats_bytes(B, L + 1) + order_bytes(B);
  return WPTV_OK;
}

namespace {

int accept_impl(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                const int32_t* firsts, const float* q, int64_t q_stride_b, int64_t q_stride_t, const int64_t* drafts,
                int64_t drafts_stride_b, const int32_t* lengths, const float* u, const float* e, float temperature,
                int top_k, int greedy, int B, int L, int V, int64_t* tokens, int32_t* n_tokens, void* workspace,
                size_t workspace_bytes, const Commit* commit, hipStream_t stream) {
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
      B, stream, scores, scores_stride_b, scores_stride_t, firsts, q, q_stride_b, q_stride_t, drafts,
      drafts_stride_b, lengths, u, e, temperature, top_k, greedy, L, V, s);
  int st = launched("accept_stats");
  if (st != WPTV_OK) return st;
  if (commit)
    hipLaunchKernelGGL(accept_pick<true>, dim3((B + 63) / 64), dim3(64), 0, stream, drafts, drafts_stride_b, lengths,
                       greedy, L, B, s, tokens, n_tokens, *commit);
  else
    hipLaunchKernelGGL(accept_pick<false>, dim3((B + 63) / 64), dim3(64), 0, stream, drafts, drafts_stride_b, lengths,
                       greedy, L, B, s, tokens, n_tokens, Commit{});
  return launched("accept_pick");
}

}  // namespace

extern "C" int wptv_accept(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                           const int32_t* firsts, const float* q, int64_t q_stride_b, int64_t q_stride_t,
                           const int64_t* drafts, int64_t drafts_stride_b, const int32_t* lengths, const float* u,
                           const float* e, float temperature, int top_k, int greedy, int B, int L, int V,
                           int64_t* tokens, int32_t* n_tokens, void* workspace, size_t workspace_bytes,
                           hipStream_t stream) {
  return accept_impl(scores, scores_stride_b, scores_stride_t, scores_dtype, firsts, q, q_stride_b, q_stride_t, drafts,
                     drafts_stride_b, lengths, u, e, temperature, top_k, greedy, B, L, V, tokens, n_tokens, workspace,
                     workspace_bytes, nullptr, stream);
}

extern "C" int wptv_accept_commit(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t,
                                  int scores_dtype, const int32_t* firsts, const float* q, int64_t q_stride_b,
                                  int64_t q_stride_t, const int64_t* drafts, int64_t drafts_stride_b,
                                  const int32_t* lengths, const float* u, const float* e, float temperature, int top_k,
                                  int greedy, int B, int L, int V, int64_t* tokens, int32_t* n_tokens,
                                  void* workspace, size_t workspace_bytes, int64_t* cache_lengths,
                                  const int64_t* cache_before, int64_t* feeds, int64_t feeds_stride, int32_t* failed,
                                  int64_t* written, hipStream_t stream) {
  if (!cache_lengths || !cache_before || !feeds)
    return fail(WPTV_E_INVALID, "accept_commit: cache_lengths, cache_before and feeds must be given");
  const Commit c{cache_lengths, cache_before, feeds, feeds_stride, failed, written};
  return accept_impl(scores, scores_stride_b, scores_stride_t, scores_dtype, firsts, q, q_stride_b, q_stride_t, drafts,
                     drafts_stride_b, lengths, u, e, temperature, top_k, greedy, B, L, V, tokens, n_tokens, workspace,
                     workspace_bytes, &c, stream);
}

namespace {

template <typename S>
void launch_order_draw(int B, hipStream_t stream, const void* scores, int64_t sb, int64_t st, const int32_t* firsts,
                       const float* q, int64_t qb, int64_t qt, const int32_t* lengths, float temperature, int top_k,
                       int L, int V, Stats s, Order o, const int64_t* drafts, int64_t db, int64_t* tokens,
                       int32_t* n_tokens, const Commit* commit) {
  const int per = (V + kSlices - 1) / kSlices;
  const int n = (per + kDT - 1) / kDT;
  const bool cut = top_k > 0 && top_k < V;
  const S* rows = static_cast<const S*>(scores);
  const dim3 grid(B * kSlices);
  const size_t lds = 4 * ((size_t)B * (L + 1) + 2 * (size_t)B * L + B);
  const Commit c = commit ? *commit : Commit{};
#define WPTV_DRAW_C(N, CU, CM)                                                                                        \
  hipLaunchKernelGGL((order_draw<N, S, CU, CM>), grid, dim3(kDT), lds, stream, rows, sb, st, firsts, q, qb, qt,     \
                     lengths, temperature, B, L, V, s, o, drafts, db, tokens, n_tokens, c)
#define WPTV_DRAW(N)                                                                                                  \
  do {                                                                                                                \
    if (cut && commit)                                                                                                \
      WPTV_DRAW_C(N, true, true);                                                                                     \
    else if (cut)                                                                                                     \
      WPTV_DRAW_C(N, true, false);                                                                                    \
    else if (commit)                                                                                                  \
      WPTV_DRAW_C(N, false, true);                                                                                    \
    else                                                                                                              \
      WPTV_DRAW_C(N, false, false);                                                                                   \
  } while (0)
  if (n <= 1) WPTV_DRAW(1);
  else if (n <= 2) WPTV_DRAW(2);
  else if (n <= 4) WPTV_DRAW(4);
  else if (n <= 8) WPTV_DRAW(8);
  else if (n <= 16) WPTV_DRAW(16);
  else WPTV_DRAW(32);
#undef WPTV_DRAW
#undef WPTV_DRAW_C
}

}  // namespace

extern "C" int wptv_accept_in_order(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t,
                                    int scores_dtype, const int32_t* firsts, const float* q, int64_t q_stride_b,
                                    int64_t q_stride_t, const int64_t* drafts, int64_t drafts_stride_b,
                                    const int32_t* lengths, const int64_t* generator_state, int64_t* next_offset,
                                    int joint, float temperature, int top_k, int B, int L, int V, int64_t* tokens,
                                    int32_t* n_tokens, void* workspace, size_t workspace_bytes,
                                    int64_t* cache_lengths, const int64_t* cache_before, int64_t* feeds,
                                    int64_t feeds_stride, int32_t* failed, int64_t* written, hipStream_t stream) {
  if (!scores || !tokens || !n_tokens || !generator_state || !next_offset || (L > 0 && (!drafts || !q)))
    return fail(WPTV_E_INVALID,
                "accept_in_order: scores, tokens, n_tokens, the generator state, next_offset (and drafts and q when "
                "L > 0) must be given");
  if (B <= 0 || L < 0 || V <= 0) return fail(WPTV_E_INVALID, "accept_in_order: bad shape B=%d L=%d V=%d", B, L, V);
  if (!(temperature > 0.f))
    return fail(WPTV_E_INVALID, "accept_in_order: temperature must be positive (got %g)", (double)temperature);
  if (joint && L != 0) return fail(WPTV_E_INVALID, "accept_in_order: a joint draw takes no drafts (L = %d)", L);
  if ((int64_t)B * (L + 1) > kScanMax || L > 64)
    return fail(WPTV_E_UNSUPPORTED, "accept_in_order: B (L + 1) = %lld above %d or L = %d above 64",
                (long long)B * (L + 1), kScanMax, L);
  if (items_for(V) == 0)
    return fail(WPTV_E_UNSUPPORTED, "accept_in_order: a vocabulary of %d is above %d", V, 64 * kT);
  if (scores_dtype != WPTV_F32 && scores_dtype != WPTV_BF16)
    return fail(WPTV_E_UNSUPPORTED, "accept_in_order: scores dtype %d is neither fp32 nor bf16", scores_dtype);
  const size_t need = stats_bytes(B, L + 1) + order_bytes(B);
  if (!workspace || workspace_bytes < need)
    return fail(WPTV_E_INVALID, "accept_in_order: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (cache_lengths && (!cache_before || !feeds))
    return fail(WPTV_E_INVALID, "accept_in_order: a commit needs cache_lengths, cache_before and feeds");
  const int cap = draw_workgroups_cap();
  if (cap <= 0) return fail(WPTV_E_HIP, "accept_in_order: the device's multiprocessors cannot be queried");
  // the multinomial's draw as torch launches it: numel entries over S threads
  const int64_t numel = joint ? (int64_t)B * V : V;
  if (numel >= (int64_t)1 << 31)
    return fail(WPTV_E_UNSUPPORTED, "accept_in_order: a joint draw of %lld entries", (long long)numel);
  const int64_t threads = 256 * std::min<int64_t>(cap, (numel + 255) / 256);
  Stats s = carve(workspace, B, L + 1);
  char* extra = static_cast<char*>(workspace) + stats_bytes(B, L + 1);
  s.arrivals = reinterpret_cast<int*>(extra);
  Order o{};
  o.state = generator_state;
  o.next = next_offset;
  o.threads = (uint32_t)threads;
  o.joint = joint ? 1 : 0;
  o.joint_step = 4 * ((numel - 1) / (4 * threads) + 1);
  o.parts = reinterpret_cast<float2*>(extra + align_up((size_t)B * 8, 256));
  (scores_dtype == WPTV_BF16 ? launch_stats<unsigned short, true> : launch_stats<float, true>)(
      B, stream, scores, scores_stride_b, scores_stride_t, firsts, q, q_stride_b, q_stride_t, drafts,
      drafts_stride_b, lengths, nullptr, nullptr, temperature, top_k, 0, L, V, s);
  int st = launched("accept_stats");
  if (st != WPTV_OK) return st;
  const Commit c{cache_lengths, cache_before, feeds, feeds_stride, failed, written};
  (scores_dtype == WPTV_BF16 ? launch_order_draw<unsigned short> : launch_order_draw<float>)(
      B, stream, scores, scores_stride_b, scores_stride_t, firsts, q, q_stride_b, q_stride_t, lengths, temperature,
      top_k, L, V, s, o, drafts, drafts_stride_b, tokens, n_tokens, cache_lengths ? &c : nullptr);
  return launched("order_draw");
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
      B, stream, scores, scores_stride_b, scores_stride_t, nullptr, nullptr, 0, 0, nullptr, 0, nullptr,
      nullptr, nullptr, 1.f, 0, 1, M - 1, V, s);
  int st = launched("accept_stats");
  if (st != WPTV_OK) return st;
  hipLaunchKernelGGL(tree_walk, dim3((B + 63) / 64), dim3(64), 0, stream, node_tokens, parents, B, M, s, path, tokens,
                     n_tokens);
  return launched("tree_walk");
}

extern "C" int wptv_greedy_tree_best(const int32_t* best, const int64_t* node_tokens, const int32_t* parents, int B,
                                     int M, int64_t* path, int64_t* tokens, int32_t* n_tokens, hipStream_t stream) {
  if (!best || !node_tokens || !parents || !path || !tokens || !n_tokens)
    return fail(WPTV_E_INVALID, "greedy_tree_best: every pointer must be given");
  if (B <= 0 || M <= 0) return fail(WPTV_E_INVALID, "greedy_tree_best: bad shape B=%d M=%d", B, M);
  Stats s{};
  s.best = const_cast<int32_t*>(best);  // the walk only reads it
  hipLaunchKernelGGL(tree_walk, dim3((B + 63) / 64), dim3(64), 0, stream, node_tokens, parents, B, M, s, path, tokens,
                     n_tokens);
  return launched("tree_walk");
}
