/* wptv.h — the C ABI of the MI355X (gfx950) speculative-decoding verify step.
 *
 * One shared library, libwptv.so, built with hipcc for gfx950 only.  Every
 * entry point is stream-ordered and asynchronous: it validates its arguments
 * on the host, enqueues kernels on `stream` and returns.  Device pointers are
 * on the current HIP device; the caller owns every buffer, the workspaces
 * included, and the library allocates nothing at run time.  Its state: a
 * per-device cache of the compute-unit count, and one file-scope device array
 * (16 MiB, present on every device the library runs on from load to exit)
 * that only wptv_verify_attention_static uses, with its address resolved once
 * per device.  Every other entry point is re-entrant across host threads
 * (calls that share a workspace on one stream are ordered by that stream).
 *
 * Status codes: WPTV_OK, or a negative WPTV_E_* value; wptv_last_error()
 * then holds a thread-local message naming the argument or the HIP error.
 *
 * Tensor layouts are row-major.  A "row" of the key/value table is the c
 * contiguous elements of one token; tables are addressed by a batch stride
 * and a row stride in elements, so the keys and values may be the two halves
 * of one (B, N, 2c) entries table, as the reference's exact layer keeps them
 * (packages/wpt-model/src/wpt_model/attention.py:184-186).
 */
#ifndef WPTV_H
#define WPTV_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WPTV_ABI_VERSION 10

enum {
  WPTV_OK = 0,
  WPTV_E_INVALID = -1,     /* a bad argument or shape */
  WPTV_E_HIP = -2,         /* a HIP runtime error (launch, device query) */
  WPTV_E_UNSUPPORTED = -3  /* a dtype, head width or feature this build has no kernel for */
};

enum { WPTV_F32 = 0, WPTV_BF16 = 1 };

/* index dtypes (counts, kept) */
enum { WPTV_I64 = 8, WPTV_I32 = 9 };

/* wptv_verify_attention flags */
enum {
  WPTV_ATTN_FORCE_GENERIC = 1,        /* run the wave-per-query VALU kernel even where the MFMA kernel applies */
  WPTV_ATTN_RANGE_FROM_POSITIONS = 2, /* read only the rows the positions reach (a table with spare capacity
                                         past its rows); by default the row-block kernel's single full-causal
                                         query group reads rows 0..N-1 and masks the ones past each query (the
                                         key-parallel kernel always reads only the rows the positions reach) */
  WPTV_ATTN_KEY_SPLIT = 4,            /* where T*H <= 80: the key-parallel MFMA kernel (each wavefront owns key
                                         tiles and holds every query row) instead of the row-block one */
  WPTV_ATTN_OUT_FM = 8,               /* the output as the output projection's operand: [B T, H c] in the
                                         fragment-major layout (below) with wptv_fm_row_blocks(B T) row blocks;
                                         bf16 row-block kernels only */
  WPTV_ATTN_ROWS32 = 16               /* head width 128: the row-block kernel on 32-row blocks (each wavefront
                                         holds 32 query rows, v_mfma_f32_32x32x16_bf16), which is the default
                                         above 128 query rows (T*H) a batch row */
};

int wptv_abi_version(void);
const char* wptv_last_error(void);

/* ---------------------------------------------------------------------------
 * Verify attention: MQA (one key/value head shared by H query heads) of the
 * k+1 (= T) query positions of each batch row against its key/value table.
 *
 * Replaces the reference's exact_attention with top_k = 0
 * (packages/wpt-model/src/wpt_model/pytorch_kernels.py:98-121,142-146, the
 * contract at :18-26, dispatched by kernels.py:160-171), its window-only
 * sparse_attention (pytorch_kernels.py:149-153,171-187,213-217 with no
 * chosen rows) and its tree-mask primitive dense_attention
 * (attention.py:74-82) with the mask "prefix plus ancestors-or-self".
 *
 *   q          [B, T, H, c] contiguous, dtype
 *   k, v       row n of batch b at k + b*k_stride_b + n*k_stride_n (elements)
 *   positions  [B, T] int64: query t of row b sees table rows
 *              max(0, p - window + 1) .. min(p, N - 1), p = positions[b, t]
 *              (window <= 0: from row 0).  A padding query past the table
 *              reads up to its last row.  NULL with a tree: query t of row
 *              b is node t, at position tree_base[b] + t.
 *   tree_base, tree_ancestors  NULL, or [B] int64 and [T] uint64: rows
 *              r >= tree_base[b] are draft-tree nodes, and query t sees node
 *              r - tree_base[b] only where that bit of tree_ancestors[t] is
 *              set (node indices < 64)
 *   sink       NULL, or [H] fp32: a per-head logit added to the softmax
 *              denominator (log-sum-exp with the scores)
 *   scale      the factor on q.k (c^-0.5 in the reference)
 *   splits     in: the number of parts each batch row's key range is cut
 *              into (0 = chosen from B, T, N and the GPU); the workspace must
 *              hold wptv_attention_workspace() bytes for the same arguments
 *   out        [B, T, H, c] contiguous, dtype
 *   lse        NULL, or [B, T, H] fp32: each query head's natural-log
 *              log-sum-exp, the sink included
 * ------------------------------------------------------------------------- */
int wptv_attention_workspace(int B, int T, int H, int c, int N, int window, int dtype, int flags,
                             int* splits, size_t* bytes);

int wptv_verify_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                          const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                          const int64_t* positions, int window, const int64_t* tree_base,
                          const uint64_t* tree_ancestors, const float* sink, int B, int T, int H, int c,
                          int N, float scale, int splits, int flags, void* out, float* lse,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

/* wptv_verify_attention_static: wptv_verify_attention with no workspace
 *   argument, for callers that cannot allocate device memory (code under HIP
 *   graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 *   has no counterpart in the reference.  The key-range parts live in a
 *   static device array of 16 MiB that each device loading the library holds
 *   until the process ends (enough for every split count the library
 *   chooses for c <= 128; a request needing more is refused with
 *   WPTV_E_INVALID and a message).  It calls no allocating routine.  Calls
 *   that overlap on one device share that array and race; calls ordered on
 *   one stream do not.  Same kernels and results as wptv_verify_attention. */
int wptv_verify_attention_static(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                                 const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                                 const int64_t* positions, int window, const int64_t* tree_base,
                                 const uint64_t* tree_ancestors, const float* sink, int B, int T, int H, int c,
                                 int N, float scale, int splits, int flags, void* out, float* lse,
                                 hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Window attention: each query at position p reads the rows of positions
 * max(0, p - window + 1) .. p, itself included and none before the text, with
 * a per-head sink in the denominator and the layer's output gate -- a window
 * layer's attention at decode (packages/wpt-model/src/wpt_model/
 * attention.py:85-107 window_attention, :142-151 WindowAttention.forward,
 * the gate of :128-130).  Where the reference reads a (B, window - 1 + T, 2c)
 * table of the carried tail and the new entries (carry.py:43-63), the table
 * here is addressed by token position:
 *   row_base NULL: a ring of ring_rows (a power of 2, >= window + T - 1) rows
 *            per batch row, position n at row n mod ring_rows (the build's
 *            window-layer cache; wptv_window_qkv_post appends to it)
 *   row_base [B] int64: position n at row n - row_base[b] of a table of
 *            ring_rows rows (the reference's tail + new table: row_base =
 *            the position of its first row)
 *   gate     NULL, or [B*T, >= H*c] in dtype (row stride gate_stride): the
 *            output is o * sigmoid(gate), each factor rounded to the dtype
 *   workspace  wptv_window_attention_workspace() bytes for the same splits
 * The T positions of a batch row are consecutive (a pass of new tokens).
 * ------------------------------------------------------------------------- */
int wptv_window_attention_workspace(int B, int T, int H, int c, int window, int dtype, int* splits, size_t* bytes);

int wptv_window_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n, const void* v,
                          int64_t v_stride_b, int64_t v_stride_n, int dtype, const int64_t* positions,
                          const int64_t* row_base, int ring_rows, int window, const float* sink, const void* gate,
                          int64_t gate_stride, int B, int T, int H, int c, float scale, int splits, void* out,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Sparse attention over chosen rows plus the last `window` rows, with a sink:
 * the reference's sparse_attention with chosen rows
 * (pytorch_kernels.py:171-187,213-217) and the sparse layer's output gate
 * (attention.py:128-130,190-): idx [B, T, K] int64, -1 = none; a row named
 * both in idx and in the window is counted twice, as the reference's
 * concatenation of the two lists counts it.  gate NULL or [B*T, >= H*c] in
 * dtype (row stride gate_stride): the output times sigmoid(gate).  bf16 with
 * head width 64 or 128 and H <= 16 runs the MFMA gather kernel (the query's
 * rows cut into `splits` parts, merged by a second kernel through the
 * workspace, wptv_sparse_attention_workspace() bytes for the same arguments);
 * anything else the wave-per-query kernel (no workspace). */
int wptv_sparse_attention_workspace(int B, int T, int H, int c, int K, int window, int N, int dtype, int* splits,
                                    size_t* bytes);

int wptv_sparse_attention(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n,
                          const void* v, int64_t v_stride_b, int64_t v_stride_n, int dtype,
                          const int64_t* idx, int K, const int64_t* positions, int window,
                          const float* sink, const void* gate, int64_t gate_stride, int B, int T, int H, int c,
                          int N, float scale, int splits, void* out, float* lse, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Exact attention's choice of rows: the top_k rows each query weighs most
 * among those at least `window` tokens back, which the sparse layers after an
 * exact layer read.  Replaces the choice of the reference's exact_attention
 * (packages/wpt-model/src/wpt_model/pytorch_kernels.py:112-117, columns
 * chosen_columns :73-77; the Triton form's _choose, triton_kernels.py:
 * 222-239,393-508).
 *
 *   q, k, positions, B, T, H, c, N, scale  as wptv_verify_attention (k rows
 *            16-byte aligned for the bf16 matrix-core path)
 *   lse      [B, T, H] fp32: each query head's natural-log log-sum-exp over
 *            the rows it sees (wptv_verify_attention's lse output)
 *   chosen   [B, T, K] int64 out, K = max(0, min(top_k, N - window)): the K
 *            rows n <= p - window (n < N) with the largest score
 *            max_h (q_h . k_n * scale - lse_h); a query with fewer such rows
 *            gets all of them, then -1.  Rows above the K-th largest score
 *            come first in row order, then rows equal to it, lowest first.
 *   workspace  wptv_choice_workspace(B, T, N) bytes (the scores)
 * H <= 128, c <= 256; nothing is launched when K = 0.
 * ------------------------------------------------------------------------- */
int wptv_choice_workspace(int B, int T, int N, size_t* bytes);

int wptv_exact_choice(const void* q, const void* k, int64_t k_stride_b, int64_t k_stride_n, int dtype,
                      const int64_t* positions, const float* lse, int B, int T, int H, int c, int N, float scale,
                      int top_k, int window, int64_t* chosen, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* ---------------------------------------------------------------------------
 * KV append: table[b, start[b] + j, :] = rows[b, j, :] for j < counts[b].
 * Replaces the scatter of the reference's Reading.everything
 * (packages/wpt-model/src/wpt_model/cache.py:110-128; the index_put at :126).
 * Rows with start[b] + j >= capacity are not written and make the call
 * fail after the fact only through the host's own check (the host keeps the
 * table large enough; the kernel never writes past capacity).
 *   table  row n of batch b at table + b*table_stride_b + n*table_stride_n
 *   rows   row j of batch b at rows + b*rows_stride_b + j*rows_stride_n
 *   width  elements per row (2c for an entries table), contiguous
 * ------------------------------------------------------------------------- */
int wptv_kv_append(void* table, int64_t table_stride_b, int64_t table_stride_n, int64_t capacity,
                   const void* rows, int64_t rows_stride_b, int64_t rows_stride_n,
                   const int64_t* start, const int64_t* counts, int B, int n, int width, int dtype,
                   hipStream_t stream);

/* wptv_cache_lengths: the cache's lengths (B,) int64 after a reading
 *   (undo = 0; the reference's Reading.finish, cache.py:130-134: before =
 *   lengths when before is not NULL, then lengths += counts) or after an undo
 *   (undo = 1; Rows.undo, cache.py:69-77: lengths = before + counts, counts
 *   being the kept tokens, a count outside 0 .. lengths - before taken as
 *   the nearest end).  counts (B,) of counts_dtype WPTV_I64 or WPTV_I32.
 *   Device-side, so that a captured step replays on the cache's state. */
int wptv_cache_lengths(int64_t* lengths, int64_t* before, const void* counts, int counts_dtype, int B, int undo,
                       hipStream_t stream);

/* wptv_next_feeds: each row's next pending token after a verify step, the
 *   last token it wrote (the reference's Writer keeps it pending for the
 *   next round, __init__.py:196-233): feeds[b * feeds_stride] =
 *   tokens[b * tokens_stride + min(counts[b], width) - 1].  A row with
 *   counts[b] < 1 (the sampler had no mass to draw from, where the
 *   reference's multinomial raises, __init__.py:219) keeps its pending token
 *   and sets *failed = 1 when failed is not NULL (the caller clears it).
 *   written: NULL, or [B] int64 running counts: written[b] += counts[b] for
 *   a row that wrote (the accepted tokens a serving loop reports, counted
 *   without a kernel of its own). */
int wptv_next_feeds(const int64_t* tokens, int64_t tokens_stride, const int* counts, int64_t* feeds,
                    int64_t feeds_stride, int B, int width, int* failed, int64_t* written, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * The decoder layer's memory-bound steps around its matrix products (the
 * reference's extend runs them as torch operations: model.py:394-436,
 * attention.py:157-188, layers.py:45-61).  dtype WPTV_F32 or WPTV_BF16 for
 * every activation; norm weights fp32; rows contiguous and 16-byte aligned.
 *
 * wptv_add_rms_norm: h [M, D] += delta (when delta is not NULL; the residual
 *   add, rounded to dtype), then y = h * rsqrt(mean(h^2) + eps) * weight in
 *   FP32 (nn.RMSNorm, layers.py:9 eps 1e-6).  D a multiple of 8, <= 4096.
 * wptv_qkv_post: the exact layer after its projection (attention.py:182-185):
 *   qkv [B*T, >= (H + 2) c] (row stride qkv_row_stride) holds q, k, v;
 *   q_out [B, T, H, c] = q_norm(q) per head; for t < counts[b] the entry
 *   [k_norm(k), v] is written at table row start[b] + t (the KV append of
 *   Reading.everything, cache.py:110-128; rows past capacity are skipped).
 * wptv_swiglu: out [M, F] = silu(gate) * up of gate_up [M, 2F] (gate first).
 * ------------------------------------------------------------------------- */
int wptv_add_rms_norm(void* h, const void* delta, const float* weight, void* y, int M, int D, int dtype, float eps,
                      hipStream_t stream);

/* wptv_add_rms_norm_parts: as wptv_add_rms_norm with delta = the sum over
 * z < splits of parts[z] (FP32 [splits, M, D], e.g. wptv_gemm_parts' output),
 * rounded to the dtype before the residual add; splits <= 8, D <= 8192.
 * y_blocks > 0: y in the fragment-major layout with that many row blocks
 * (bf16, D a multiple of 32, M <= 16 y_blocks; the operand of
 * wptv_gemm_fm_*); 0: row-major.  Likewise for wptv_embed_rms_norm. */
/* wptv_embed_rms_norm: the first layer's input (model.py:394-400: the
 *   embedding of ids, then the first attention norm): h [M, D] =
 *   table[ids[m]] (ids clamped into [0, vocab)), y = RMSNorm(h) * weight as
 *   wptv_add_rms_norm; with positions (not NULL) also positions[m] =
 *   lengths[m / T] + m % T, each token's place after its row's earlier ones
 *   (Place.positions, sequence.py:70-73). */
int wptv_embed_rms_norm(const int64_t* ids, const void* table, int64_t vocab, const float* weight, void* h, void* y,
                        int y_blocks, int M, int D, int dtype, float eps, const int64_t* lengths, int64_t* positions,
                        int T, hipStream_t stream);

int wptv_add_rms_norm_parts(void* h, const float* parts, int splits, const float* weight, void* y, int y_blocks,
                            int M, int D, int dtype, float eps, hipStream_t stream);

int wptv_qkv_post(const void* qkv, int64_t qkv_row_stride, const float* q_norm, const float* k_norm, void* q_out,
                  void* table, int64_t table_stride_b, int64_t table_stride_n, int64_t capacity,
                  const int64_t* start, const int64_t* counts, int B, int T, int H, int c, int dtype, float eps,
                  hipStream_t stream);

/* wptv_qkv_post_parts: as wptv_qkv_post with the projection given as FP32
 * split-K parts [splits, B*T, (H + 2) c] (wptv_gemm_parts' output), summed and
 * rounded to the dtype first; splits <= 8. */
int wptv_qkv_post_parts(const float* parts, int splits, const float* q_norm, const float* k_norm, void* q_out,
                        void* table, int64_t table_stride_b, int64_t table_stride_n, int64_t capacity,
                        const int64_t* start, const int64_t* counts, int B, int T, int H, int c, int dtype, float eps,
                        hipStream_t stream);

/* wptv_window_qkv_post: a window layer after its projection (attention.py:
 *   113-135 queries / entries): as wptv_qkv_post, then the last rope_dims
 *   dimensions of each normed query head and key turned by the token's
 *   position p = start[b] + t (rotate, attention.py:59-71: adjacent pairs
 *   (2i, 2i + 1) by the angle p / rope_div[i], in FP32 from the normed values
 *   rounded to the dtype); rope_div [rope_dims / 2] fp32 on the device, the
 *   reference's base^(2i / rope_dims); the entry [rotate(k_norm(k)), v] of
 *   t < counts[b] written at ring row (start[b] + t) mod ring_rows (a power
 *   of 2). */
int wptv_window_qkv_post(const void* qkv, int64_t qkv_row_stride, const float* q_norm, const float* k_norm,
                         void* q_out, void* ring, int64_t ring_stride_b, int64_t ring_stride_n, int ring_rows,
                         const int64_t* start, const int64_t* counts, int B, int T, int H, int c, int rope_dims,
                         const float* rope_div, int dtype, float eps, hipStream_t stream);

/* wptv_heads_rms_norm: a sparse layer's query norm (attention.py:191-216:
 *   q_norm(q(x)) per head): out [rows, H, c] = RMSNorm of each head of x
 *   (row r at x + r*row_stride) times weight [c], in FP32. */
int wptv_heads_rms_norm(const void* x, int64_t row_stride, const float* weight, void* out, int rows, int H, int c,
                        int dtype, float eps, hipStream_t stream);

/* wptv_heads_rms_norm_rope: a window attention's query and key
 *   (packages/wpt-model/src/wpt_model/attention.py:130-136:
 *   rotate(q_norm(q(x)), positions), rotate(k_norm(k(x)), positions)):
 *   wptv_heads_rms_norm, then the last rope_dims (even, <= c) values of each
 *   head of row r turned by positions[r] (rotate, attention.py:59-71: pairs
 *   (2i, 2i + 1) by the angle positions[r] / rope_div[i], in FP32 from the
 *   normed values rounded to the dtype).  rope_div [rope_dims / 2] FP32. */
int wptv_heads_rms_norm_rope(const void* x, int64_t row_stride, const float* weight, void* out, int rows, int H,
                             int c, int dtype, float eps, const int64_t* positions, int rope_dims,
                             const float* rope_div, hipStream_t stream);

int wptv_swiglu(const void* gate_up, void* out, int M, int F, int dtype, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Matrix products on the matrix cores: out[M, N] = x[M, K] . w[N, K]^T in
 * bf16 with FP32 accumulation -- the reference's nn.Linear projections and
 * lm_head under bf16 autocast (packages/wpt-model/src/wpt_model/
 * attention.py:113-124,157-168, layers.py:45-61, model.py:267,471): the
 * skinny products at the verify step's few rows (M <= 512; N a multiple of
 * 64, K of 64), and with splits 0 above 320 rows the 256 x 256 tiles (any
 * M; N a multiple of 256, K of 32; no workspace).
 *
 *   x, w       row-major bf16 with leading dimensions ldx, ldw (elements)
 *   out        [M, N] with leading dimension ldo: bf16 (out_dtype
 *              WPTV_BF16) or FP32 holding the bf16-rounded product
 *              (WPTV_F32: the reference's bf16 logits cast to FP32)
 *   splits     parts of K (0 = chosen from M, N, K and the GPU); the FP32
 *              part products go through the workspace,
 *              wptv_gemm_workspace() bytes for the same M, N, K and splits
 * ------------------------------------------------------------------------- */
int wptv_gemm_workspace(int M, int N, int K, int* splits, size_t* bytes);

int wptv_gemm(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out, int64_t ldo,
              int out_dtype, int splits, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* wptv_gemm_parts: the split products only, FP32 parts [splits, M, N] (each
 * the product over one part of K; their sum is x . w^T), for a consumer that
 * sums them itself (wptv_add_rms_norm_parts); splits as wptv_gemm_workspace
 * returns it. */
int wptv_gemm_parts(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, int splits,
                    float* parts, size_t parts_bytes, hipStream_t stream);

/* wptv_gemm_swiglu: the feed-forward block's gate/up product with SwiGLU in
 * its epilogue (layers.py:45-61: silu(gate(x)) * up(x)), one part of K:
 * out bf16 [M, N / 2] (leading dimension ldo) = silu(g) * u of the product's
 * bf16-rounded gate g and up u, rounded once (the values wptv_gemm then
 * wptv_swiglu give).  w holds the gate and up rows interleaved by tiles of
 * 64: rows 64 t .. 64 t + 31 are the gate rows of features 32 t .. 32 t + 31,
 * rows 64 t + 32 .. 64 t + 63 their up rows (N a multiple of 64). */
int wptv_gemm_swiglu(const void* x, int64_t ldx, const void* w, int64_t ldw, int M, int N, int K, void* out,
                     int64_t ldo, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * The same products with fragment-major ("fm") operands, for the verify
 * step's projections at M <= 160 rows (the reference's nn.Linear under bf16
 * autocast: attention.py:157-168, layers.py:45-61).  An fm matrix A [R, K]
 * (bf16, K a multiple of 32) is stored as 1 KiB blocks of 16 rows x 32
 * columns: block (ks, rb) at element (ks * RB + rb) * 512, RB its row-block
 * count, and in it element 8 l + e holds A[16 rb + l % 16][32 ks + 8 (l / 16)
 * + e] (l < 64, e < 8; rows past R are padding): the register order of the
 * bf16 16x16x32 matrix instruction, so a wavefront reads a block as 1 KiB of
 * contiguous memory.  Weights are packed once (RB = N / 16); X holds
 * wptv_fm_row_blocks(M) row blocks and is written in that layout by its
 * producer (wptv_add_rms_norm_parts, wptv_embed_rms_norm, wptv_verify_attention
 * with WPTV_ATTN_OUT_FM, wptv_gemm_fm_swiglu).  No counterpart in the
 * reference: a layout of this build's own.
 *
 * wptv_fm_pack: out = a [rows, K] (row-major bf16, leading dimension lda) in
 *   the fm layout with row_blocks row blocks, padding rows zero.
 * wptv_fm_row_blocks: the row blocks an fm X of M rows has (2 ceil(M / 32)).
 * wptv_gemm_fm_plan: the part count of a product (*splits 0: chosen; in: a
 *   count to check) and the bytes of its FP32 parts; swiglu: the gate/up
 *   form (one part).  N a multiple of 32 (64 for swiglu), K of 128.
 * wptv_gemm_fm_parts: parts [splits, M, N] FP32 of x . w^T, each over one
 *   part of K, for a consumer that sums them (wptv_qkv_post_parts,
 *   wptv_add_rms_norm_parts).
 * wptv_gemm_fm_swiglu: the gate/up product (w's rows interleaved by tiles of
 *   64 as for wptv_gemm_swiglu, then packed) with SwiGLU in its epilogue:
 *   out_fm [M, N / 2] bf16 in the fm layout with wptv_fm_row_blocks(M) row
 *   blocks (the down product's X).
 * ------------------------------------------------------------------------- */
int wptv_fm_pack(const void* a, int64_t lda, int rows, int K, int row_blocks, void* out, hipStream_t stream);

int wptv_fm_row_blocks(int M);

int wptv_gemm_fm_plan(int M, int N, int K, int swiglu, int* splits, size_t* parts_bytes);

int wptv_gemm_fm_parts(const void* x_fm, const void* w_fm, int M, int N, int K, int splits, float* parts,
                       size_t parts_bytes, hipStream_t stream);

int wptv_gemm_fm_swiglu(const void* x_fm, const void* w_fm, int M, int N, int K, void* out_fm, hipStream_t stream);

/* wptv_gemm_fm_wide: out [M, N] = x . w^T over many rows -- the lm_head of a
 *   reading wider than the skinny products serve (model.py:471 under bf16
 *   autocast: the tree verification's 16 x 31 = 496 node rows against the
 *   [32768 x 2048] head) -- on 256 x 256 output tiles, one workgroup of eight
 *   wavefronts each.  x_fm: fm with x_blocks >= wptv_fm_row_blocks(M) row
 *   blocks; w_fm: fm with N / 16 row blocks (wptv_fm_pack); N a multiple of
 *   256, K of 32.  out: bf16 (out_dtype WPTV_BF16) or FP32 holding the
 *   bf16-rounded product (WPTV_F32, the reference's .float() of the bf16
 *   logits), leading dimension ldo (a multiple of 8, >= N).  One pass, no
 *   workspace. */
int wptv_gemm_fm_wide(const void* x_fm, int x_blocks, const void* w_fm, int M, int N, int K, void* out, int64_t ldo,
                      int out_dtype, hipStream_t stream);

/* wptv_gemm_fm_wide_argmax: the greedy decisions' per-row argmax of that
 *   product without storing it: best[m] = the first index of the largest
 *   bf16-rounded value of row m of x . w^T (torch.argmax of the reference's
 *   bf16 logits, model.py:471, as its greedy verification reads them:
 *   packages/wpt-worker/src/wpt_worker/evaluation.py:74-81: a NaN counts
 *   as the largest value, the first of several).  The 256 x 256 tiles' epilogue keeps each
 *   row's (maximum, index) over its columns in the workspace
 *   (wptv_gemm_fm_wide_argmax_workspace bytes: 8 (N / 256) M), a second
 *   kernel reduces them in column order.  Shapes as wptv_gemm_fm_wide. */
int wptv_gemm_fm_wide_argmax_workspace(int M, int N, size_t* bytes);

int wptv_gemm_fm_wide_argmax(const void* x_fm, int x_blocks, const void* w_fm, int M, int N, int K, int32_t* best,
                             void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Acceptance: the reference's per-row verification loop of
 * Writer._speculate (packages/wpt-inference/src/wpt_inference/__init__.py:
 * 210-229) with its sampling distribution Writer._probabilities (:173-179),
 * fused over the vocabulary for every row at once.
 *
 *   scores   position j (0..L) of row b at scores + b*scores_stride_b +
 *            (firsts[b] + j)*scores_stride_t (in elements), V contiguous
 *            values of scores_dtype (WPTV_F32, or WPTV_BF16: the lm_head's
 *            logits as they come, read as their exact FP32 values, which is
 *            the reference's scores.float(), :174): the model's scores at the
 *            pending token and at each draft (the reference's
 *            scores[i, firsts:firsts + L + 1], :210-212)
 *   firsts   NULL (0 for every row) or [B] int32
 *   q        draft distributions, position j (0..L-1) of row b at
 *            q + b*q_stride_b + j*q_stride_t, V contiguous fp32
 *   drafts   [B, L] int64 (row stride drafts_stride_b)
 *   lengths  NULL (every row verifies L drafts) or [B] int32 in 0..L (a
 *            length outside it is taken as the nearest end)
 *   u        [B, L] fp32 uniforms in [0, 1): draft j of row b is kept iff
 *            u[b, j] * q[b, j, draft] < p[j, draft]
 *   e        [B, V] fp32 Exp(1) draws: the replacement or bonus token is
 *            argmax_v w_v / e[b, v], w the distribution it is drawn from
 *            (the reference's multinomial draw of one token)
 *   temperature, top_k  the reference's (top_k <= 0 or >= V: no cut)
 *   greedy   1: greedy verification instead (q, u, e unused and may be
 *            NULL): a draft is kept iff it is the first maximal index of its
 *            position's scores (torch.argmax's: a NaN counts as the largest
 *            value), and the replacement or bonus is that index
 *   tokens   [B, L + 1] int64 out: the kept drafts, then the drawn token;
 *            entries past n_tokens[b] are -1
 *   n_tokens [B] int32 out: kept drafts + 1; -1 for a row whose residual
 *            distribution max(0, p - q) has no mass (the reference raises)
 *   workspace  wptv_accept_workspace(B, L) bytes
 * Rows and positions are independent; the vocabulary may hold up to 65536
 * entries.
 * ------------------------------------------------------------------------- */
int wptv_accept_workspace(int B, int L, size_t* bytes);

int wptv_accept(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                const int32_t* firsts, const float* q, int64_t q_stride_b, int64_t q_stride_t, const int64_t* drafts,
                int64_t drafts_stride_b, const int32_t* lengths, const float* u, const float* e, float temperature,
                int top_k, int greedy, int B, int L, int V, int64_t* tokens, int32_t* n_tokens, void* workspace,
                size_t workspace_bytes, hipStream_t stream);

/* wptv_accept_commit: wptv_accept, and in the same launch as the pick, what
 *   the verify step does next with each row's count n = n_tokens[b] (the
 *   reference's Writer._speculate, __init__.py:196-233, after the sampler):
 *   the cache takes back the rejected drafts (WPT.undo / Rows.undo,
 *   model.py:475-483, cache.py:69-77): cache_lengths[b] = cache_before[b] +
 *   n, n taken into 0 .. cache_lengths[b] - cache_before[b]; then, as
 *   wptv_next_feeds with tokens and n_tokens, the last written token becomes
 *   feeds[b * feeds_stride], a row with n < 1 keeps its pending token and
 *   sets *failed = 1 (failed may be NULL), and written[b] += n (written may
 *   be NULL).  The same results as wptv_accept, wptv_cache_lengths (undo) and
 *   wptv_next_feeds in turn, in two launches instead of four.
 *   cache_lengths, cache_before [B] int64; feeds int64. */
int wptv_accept_commit(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                       const int32_t* firsts, const float* q, int64_t q_stride_b, int64_t q_stride_t,
                       const int64_t* drafts, int64_t drafts_stride_b, const int32_t* lengths, const float* u,
                       const float* e, float temperature, int top_k, int greedy, int B, int L, int V, int64_t* tokens,
                       int32_t* n_tokens, void* workspace, size_t workspace_bytes, int64_t* cache_lengths,
                       const int64_t* cache_before, int64_t* feeds, int64_t feeds_stride, int32_t* failed,
                       int64_t* written, hipStream_t stream);

/* wptv_accept_in_order: wptv_accept (with wptv_accept_commit's moves when
 *   cache_lengths is not NULL) drawing as the reference's loop draws from a
 *   torch generator on this device, in its order (Writer._speculate,
 *   __init__.py:214-229): row by row, one torch.rand(()) per draft it judges,
 *   then one torch.multinomial(w, 1) over the vocabulary; or, with joint = 1
 *   and L = 0, one torch.multinomial of every row's distribution at once
 *   (Writer._sample, :181-182).  No tape: the draws are torch's Philox4x32-10
 *   stream itself (torch's device generator through hipRAND).
 *   generator_state  [2] int64 on the device: the generator's seed and
 *                    offset (its get_state())
 *   next_offset      int64 on the device out: the offset after these draws
 *                    (may be generator_state + 1); set it back on the
 *                    generator to continue its stream
 *   the rest as wptv_accept (u and e replaced by the two above; greedy is
 *   not taken: a greedy step draws nothing) and wptv_accept_commit (all of
 *   cache_lengths, cache_before, feeds, failed, written may be NULL).
 *   B (L + 1) <= 3072, L <= 64; workspace wptv_accept_workspace(B, L) bytes.
 *   Two launches: the statistics, then the draws (the loop's uniforms
 *   replayed to find each row's first rejection; the multinomial's
 *   exponentials over 32 slices of the vocabulary a row), whose last slice
 *   of a row to finish makes that row's pick.  Calls that share a workspace
 *   must not overlap. */
int wptv_accept_in_order(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                         const int32_t* firsts, const float* q, int64_t q_stride_b, int64_t q_stride_t,
                         const int64_t* drafts, int64_t drafts_stride_b, const int32_t* lengths,
                         const int64_t* generator_state, int64_t* next_offset, int joint, float temperature, int top_k,
                         int B, int L, int V, int64_t* tokens, int32_t* n_tokens, void* workspace,
                         size_t workspace_bytes, int64_t* cache_lengths, const int64_t* cache_before, int64_t* feeds,
                         int64_t feeds_stride, int32_t* failed, int64_t* written, hipStream_t stream);

/* Greedy verification of a draft tree of M nodes per row (node 0 the root,
 * the token already written; parents[i] < i, parents[0] = -1): from the root,
 * move to the child whose token equals the argmax (first maximal index) of
 * the current node's scores, the lowest node index among equal children,
 * until none does; then the argmax.  Scores position i = node i (row stride
 * scores_stride_b, node stride scores_stride_t, V contiguous values of
 * scores_dtype, WPTV_F32 or WPTV_BF16);
 * node_tokens [B, M] int64; parents [M] int32.
 *   path     [B, M + 1] int64 out: the accepted node indices from the root
 *            (the root included), -1 after
 *   tokens   [B, M + 1] int64 out: the accepted nodes' tokens after the
 *            root, then the argmax; -1 after
 *   n_tokens [B] int32 out: accepted nodes after the root + 1 (each
 *            node's argmax in torch.argmax's order, a NaN the largest)
 *   workspace  wptv_accept_workspace(B, M - 1) bytes */
int wptv_greedy_tree(const void* scores, int64_t scores_stride_b, int64_t scores_stride_t, int scores_dtype,
                     const int64_t* node_tokens, const int32_t* parents, int B, int M, int V, int64_t* path,
                     int64_t* tokens, int32_t* n_tokens, void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* wptv_greedy_tree_best: the same walk from each node's argmax already
 *   found (best [B, M] int32: for instance wptv_gemm_fm_wide_argmax of the
 *   nodes' lm_head rows; a node whose best is -1 ends the walk writing
 *   nothing, n_tokens -1). */
int wptv_greedy_tree_best(const int32_t* best, const int64_t* node_tokens, const int32_t* parents, int B, int M,
                          int64_t* path, int64_t* tokens, int32_t* n_tokens, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* WPTV_H */
