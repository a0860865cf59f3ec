// The in-place KV append of the generation cache: each row's new entries are
// written after its earlier ones (the scatter of the reference's
// Reading.everything, packages/wpt-model/src/wpt_model/cache.py:110-128,
// held[row, first[row] + j] = new[row, j] for j < counts[row]).
//
// One thread moves 16 bytes; rows are contiguous, so a wavefront moves
// 1 KiB of consecutive row bytes.  HBM-bound: B * n * width * elem bytes
// read and written.
#include "wptv_common.h"

namespace wptv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void kv_append_16(unsigned char* __restrict__ table, int64_t tsb, int64_t tsn,
                                                    int64_t capacity, const unsigned char* __restrict__ rows,
                                                    int64_t rsb, int64_t rsn, const int64_t* __restrict__ start,
                                                    const int64_t* __restrict__ counts, int n, int row_chunks) {
  const int b = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * row_chunks) return;
  const int j = (int)(idx / row_chunks);
  const int chunk = (int)(idx % row_chunks);
  if (j >= counts[b]) return;
  const int64_t dst_row = start[b] + j;
  if (dst_row < 0 || dst_row >= capacity) return;  // never past the table
  const u32x4* src = reinterpret_cast<const u32x4*>(rows + b * rsb + j * rsn) + chunk;
  u32x4* dst = reinterpret_cast<u32x4*>(table + b * tsb + dst_row * tsn) + chunk;
  *dst = *src;
}

// The cache's lengths after a reading (the reference's Reading.finish,
// cache.py:130-139: before = lengths when the reading can be undone, lengths
// += counts) or after an undo (Rows.undo, cache.py:69-77: lengths = before +
// kept); counts / kept int64 or int32.  One thread per batch row.
template <typename C>
__global__ __launch_bounds__(64) void cache_lengths(int64_t* __restrict__ lengths, int64_t* __restrict__ before,
                                                    const C* __restrict__ counts, int B, int undo) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int64_t n = (int64_t)counts[b];
  if (undo) {
    // kept tokens outside 0 .. the tokens read (a row the sampler could not
    // draw for writes -1) are taken as the nearest end
    const int64_t start = before[b], read = lengths[b] - start;
    lengths[b] = start + min(max(n, (int64_t)0), read);
  } else {
    const int64_t len = lengths[b];
    if (before) before[b] = len;
    lengths[b] = len + n;
  }
}

// Each row's next pending token after a verify step: the last token it wrote,
// tokens[b, counts[b] - 1], into feeds[b, 0].  A row that wrote nothing (a
// count below 1: the sampler found no mass to draw from) keeps its pending
// token and raises *failed (when given) for the host to report.
__global__ __launch_bounds__(64) void next_feeds(const int64_t* __restrict__ tokens, int64_t tokens_stride,
                                                 const int* __restrict__ counts, int64_t* __restrict__ feeds,
                                                 int64_t feeds_stride, int B, int width, int* __restrict__ failed,
                                                 int64_t* __restrict__ written) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int n = counts[b];
  if (n < 1) {
    if (failed) *failed = 1;
    return;
  }
  feeds[(int64_t)b * feeds_stride] = tokens[(int64_t)b * tokens_stride + min(n, width) - 1];
  if (written) written[b] += n;
}

// Byte-wise form for rows whose size or strides are not multiples of 16 bytes.
__global__ __launch_bounds__(256) void kv_append_bytes(unsigned char* __restrict__ table, int64_t tsb, int64_t tsn,
                                                       int64_t capacity, const unsigned char* __restrict__ rows,
                                                       int64_t rsb, int64_t rsn, const int64_t* __restrict__ start,
                                                       const int64_t* __restrict__ counts, int n, int row_bytes) {
  const int b = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * row_bytes) return;
  const int j = (int)(idx / row_bytes);
  const int byte = (int)(idx % row_bytes);
  if (j >= counts[b]) return;
  const int64_t dst_row = start[b] + j;
  if (dst_row < 0 || dst_row >= capacity) return;
  table[b * tsb + dst_row * tsn + byte] = rows[b * rsb + j * rsn + byte];
}

}  // namespace
}  // namespace wptv

using namespace wptv;

extern "C" int wptv_kv_append(void* table, int64_t table_stride_b, int64_t table_stride_n, int64_t capacity,
                              const void* rows, int64_t rows_stride_b, int64_t rows_stride_n, const int64_t* start,
                              const int64_t* counts, int B, int n, int width, int dtype, hipStream_t stream) {
  if (!table || !rows || !start || !counts)
    return fail(WPTV_E_INVALID, "kv_append: table, rows, start and counts must be given");
  if (B < 0 || n < 0 || width <= 0 || capacity < 0)
    return fail(WPTV_E_INVALID, "kv_append: bad shape B=%d n=%d width=%d capacity=%lld", B, n, width,
                (long long)capacity);
  if (dtype != WPTV_F32 && dtype != WPTV_BF16)
    return fail(WPTV_E_UNSUPPORTED, "kv_append: dtype %d is neither fp32 nor bf16", dtype);
  if (table_stride_n < width || rows_stride_n < width)
    return fail(WPTV_E_INVALID, "kv_append: a row stride below the row width");
  if (B == 0 || n == 0) return WPTV_OK;
  const int64_t elem = dtype == WPTV_F32 ? 4 : 2;
  const int64_t row_bytes = width * elem;
  const int64_t tsb = table_stride_b * elem, tsn = table_stride_n * elem;
  const int64_t rsb = rows_stride_b * elem, rsn = rows_stride_n * elem;
  const bool wide = row_bytes % 16 == 0 && tsb % 16 == 0 && tsn % 16 == 0 && rsb % 16 == 0 && rsn % 16 == 0 &&
                    aligned(table, 16) && aligned(rows, 16);
  const int threads = 256;
  if (wide) {
    const int row_chunks = (int)(row_bytes / 16);
    const int64_t total = (int64_t)n * row_chunks;
    dim3 grid((unsigned)((total + threads - 1) / threads), B);
    hipLaunchKernelGGL(kv_append_16, grid, dim3(threads), 0, stream, static_cast<unsigned char*>(table), tsb, tsn,
                       capacity, static_cast<const unsigned char*>(rows), rsb, rsn, start, counts, n, row_chunks);
    return launched("kv_append_16");
  }
  const int64_t total = (int64_t)n * row_bytes;
  dim3 grid((unsigned)((total + threads - 1) / threads), B);
  hipLaunchKernelGGL(kv_append_bytes, grid, dim3(threads), 0, stream, static_cast<unsigned char*>(table), tsb, tsn,
                     capacity, static_cast<const unsigned char*>(rows), rsb, rsn, start, counts, n, (int)row_bytes);
  return launched("kv_append_bytes");
}

extern "C" int wptv_cache_lengths(int64_t* lengths, int64_t* before, const void* counts, int counts_dtype, int B,
                                  int undo, hipStream_t stream) {
  if (!lengths || !counts || (undo && !before))
    return fail(WPTV_E_INVALID, "cache_lengths: lengths and counts (and before, to undo) must be given");
  if (B < 0) return fail(WPTV_E_INVALID, "cache_lengths: B = %d", B);
  if (B == 0) return WPTV_OK;
  dim3 grid((unsigned)((B + 63) / 64));
  if (counts_dtype == WPTV_I64)
    hipLaunchKernelGGL(cache_lengths<int64_t>, grid, dim3(64), 0, stream, lengths, before,
                       static_cast<const int64_t*>(counts), B, undo);
  else if (counts_dtype == WPTV_I32)
    hipLaunchKernelGGL(cache_lengths<int>, grid, dim3(64), 0, stream, lengths, before,
                       static_cast<const int*>(counts), B, undo);
  else
    return fail(WPTV_E_UNSUPPORTED, "cache_lengths: counts of dtype %d are neither int64 nor int32", counts_dtype);
  return launched("cache_lengths");
}

extern "C" int wptv_next_feeds(const int64_t* tokens, int64_t tokens_stride, const int* counts, int64_t* feeds,
                               int64_t feeds_stride, int B, int width, int* failed, int64_t* written,
                               hipStream_t stream) {
  if (!tokens || !counts || !feeds) return fail(WPTV_E_INVALID, "next_feeds: every pointer must be given");
  if (B < 0 || width <= 0 || tokens_stride < width)
    return fail(WPTV_E_INVALID, "next_feeds: bad shape B=%d width=%d stride=%lld", B, width, (long long)tokens_stride);
  if (B == 0) return WPTV_OK;
  hipLaunchKernelGGL(next_feeds, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, stream, tokens, tokens_stride, counts,
                     feeds, feeds_stride, B, width, failed, written);
  return launched("next_feeds");
}
