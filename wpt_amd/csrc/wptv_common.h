// Shared helpers of libwptv: status reporting, device queries, bf16 and
// wavefront utilities for gfx950 (64-wide wavefronts).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "../../include/wptv.h"

namespace wptv {

// Sets the calling thread's last-error message and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// WPTV_OK when the last launch on this thread succeeded, else WPTV_E_HIP.
int launched(const char* kernel);

// Compute units of the current device (cached per device).
int compute_units();

// The most workgroups torch's distribution kernels launch on the current
// device: multiprocessors x (max threads a multiprocessor / 256); -1 when
// the device cannot be queried (cached per device).
int draw_workgroups_cap();

// The wide-tile product (gemm_wide.hip): out[M, N] = x . w^T on 256 x 256
// tiles, for readings of more rows than the skinny products take.
bool gemm_wide_fits(int M, int N, int K);
int gemm_wide(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out, int64_t ldo,
              int out_dtype, hipStream_t stream);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---- device-side helpers -------------------------------------------------

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_to_f32(unsigned short h) {
  return __uint_as_float(static_cast<unsigned int>(h) << 16);
}

// Round to nearest even, as torch's float -> bfloat16 conversion does (NaN kept quiet).
__device__ __forceinline__ unsigned short f32_to_bf16(float f) {
  unsigned int u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<unsigned short>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<unsigned short>(u >> 16);
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_f32<unsigned short>(const unsigned short* p) { return bf16_to_f32(*p); }

template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) { return f; }
template <>
__device__ __forceinline__ unsigned short from_f32<unsigned short>(float f) { return f32_to_bf16(f); }

// f rounded to the element type T and read back.
template <typename T>
__device__ __forceinline__ float rounded(float f);
template <>
__device__ __forceinline__ float rounded<float>(float f) { return f; }
template <>
__device__ __forceinline__ float rounded<unsigned short>(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// An order-preserving unsigned key of a float (larger float, larger key;
// -0 below +0), and its inverse: radix selection runs on these keys.
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}


// ---- lane exchanges without LDS traffic -------------------------------------

// DPP moves within a 16-lane row: lane i takes lane i ^ 1, i ^ 2 (quad
// permutes), 7 - i within its half-row, 15 - i within its row.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_move(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}

// The max over the 16 lanes of a row, in every lane of it.
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, __int_as_float(dpp_move<kDppXor1>(__float_as_int(x))));
  x = fmaxf(x, __int_as_float(dpp_move<kDppXor2>(__float_as_int(x))));
  x = fmaxf(x, __int_as_float(dpp_move<kDppHalfMirror>(__float_as_int(x))));
  return fmaxf(x, __int_as_float(dpp_move<kDppMirror>(__float_as_int(x))));
}

// The sum over the 64 lanes of a wavefront, in every lane, without LDS
// traffic (wave_sum's shuffles are six dependent ds_bpermute round trips):
// pairs, quads, 8 and 16 lanes by DPP, then the rows by permlane swaps.  Each
// step adds two equal-count partial sums, so every lane ends with the same bits.
// The DPP and permlane moves read inactive lanes' registers as they stand, so
// a wavefront with lanes off (a row narrower than 64 lanes) takes wave_sum.
__device__ __forceinline__ float wave_sum_dpp(float x) {
  if (__builtin_amdgcn_read_exec() != ~0ull) return wave_sum(x);
  x += __int_as_float(dpp_move<kDppXor1>(__float_as_int(x)));
  x += __int_as_float(dpp_move<kDppXor2>(__float_as_int(x)));
  x += __int_as_float(dpp_move<kDppHalfMirror>(__float_as_int(x)));
  x += __int_as_float(dpp_move<kDppMirror>(__float_as_int(x)));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The minimum and the maximum over the 64 lanes of a wavefront, in every lane
// (DPP within rows, permlane swaps across them); every lane must be active.
__device__ __forceinline__ int wave_min_i32(int x) {
  x = min(x, dpp_move<kDppXor1>(x));
  x = min(x, dpp_move<kDppXor2>(x));
  x = min(x, dpp_move<kDppHalfMirror>(x));
  x = min(x, dpp_move<kDppMirror>(x));
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = min((int)a[0], (int)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return min((int)b[0], (int)b[1]);
}

__device__ __forceinline__ int wave_max_i32(int x) {
  x = max(x, dpp_move<kDppXor1>(x));
  x = max(x, dpp_move<kDppXor2>(x));
  x = max(x, dpp_move<kDppHalfMirror>(x));
  x = max(x, dpp_move<kDppMirror>(x));
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = max((int)a[0], (int)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return max((int)b[0], (int)b[1]);
}

// The sum over the 64 lanes of a wavefront, in every lane: the rows by DPP,
// then across the four rows by permlane swaps.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t x) {
  x += (uint32_t)dpp_move<kDppXor1>((int)x);
  x += (uint32_t)dpp_move<kDppXor2>((int)x);
  x += (uint32_t)dpp_move<kDppHalfMirror>((int)x);
  x += (uint32_t)dpp_move<kDppMirror>((int)x);
  const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = a[0] + a[1];
  const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return b[0] + b[1];
}

// ---- fragment-major ("fm") operands ------------------------------------------
//
// A bf16 matrix A [R, K] stored as 1 KiB blocks of 16 rows x 32 columns: block
// (ks, rb) -- rows 16 rb .. 16 rb + 15, columns 32 ks .. 32 ks + 31 -- at
// element (ks * RB + rb) * 512, RB the blocks' row count (rows past R are
// padding); in it lane l = 16 g + j holds row 16 rb + j, columns 32 ks + 8 g
// .. + 7 (8 elements, 16 bytes).  That is the operand layout of
// v_mfma_f32_16x16x32_bf16 (A and B alike), so one 16-byte load per lane
// reads a block, 1 KiB contiguous.  8 consecutive columns from a multiple of
// 8 (4 from a multiple of 4) are contiguous.
__device__ __forceinline__ int64_t fm_offset(int r, int k, int rb_count) {
  return ((int64_t)((k >> 5) * rb_count + (r >> 4)) * 64 + (((k >> 3) & 3) << 4) + (r & 15)) * 8 + (k & 7);
}

// The row blocks an fm operand of M rows is stored with: an even count,
// 2 ceil(M / 32), so that a few kernel forms serve every row count.
__host__ __device__ __forceinline__ int fm_row_blocks(int M) { return 2 * ((M + 31) / 32); }

// ---- LDS DMA (global -> LDS without registers) -----------------------------

// s_waitcnt with vmcnt = n and the other counters left alone (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
  asm volatile("" ::: "memory");
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
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

// The same for data read once (non-temporal: no cache line kept for reuse).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_16B_nt(i32x4 rsrc, uint32_t voffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Global -> LDS copy of 16 bytes per lane at base + soffset + voffset
// (soffset uniform): lane l's bytes land at LDS byte address `lds` + 16 l.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_16B_at(i32x4 rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(soffset), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace wptv
