"""Python entry points of libwptv's decoder-layer kernels (include/wptv.h):
the residual add + RMSNorm, the exact layer's q/k norms + KV append, the
window layer's q/k norms + rotary encoding + ring append, and SwiGLU, each one pass over its rows on the GPU (the reference runs them as
separate torch operations: model.py:394-436, attention.py:157-188,
layers.py:45-61)."""

import torch

from . import _lib
from ._lib import KernelUnavailable, check, ptr

EPS = 1e-6
LINEAR_MAX_ROWS = 512  # rows wptv_gemm's skinny products take
WIDE_MIN_ROWS = 321   # from here an unsplit wptv_gemm runs on the 256 x 256 tiles


def _gpu(*tensors):
    for x in tensors:
        if x is not None and x.device.type != "cuda":
            raise KernelUnavailable(f"the HIP layer kernels run on a GPU; a tensor is on {x.device}")


def _rows(x, name):
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return x


def embed_rms_norm(ids, table, weight, h, y, lengths=None, positions=None, eps=EPS, fm=False):
    """h = table[ids] (ids (B, T) int64 on the device, clamped into the
    vocabulary), y = RMSNorm(h) * weight; with lengths (B,) and positions
    (B, T) int64 also positions = lengths[:, None] + t.  fm: y is a flat
    fragment-major operand of B T rows (fm_empty), not (B, T, D)."""
    _gpu(table, weight, h, y)
    B, T = ids.shape
    V, D = table.shape
    if h.shape != (B, T, D) or h.dtype != table.dtype or y.dtype != table.dtype:
        raise ValueError(f"h must be (B={B}, T={T}, D={D}) and y in the table's dtype")
    y_blocks = _fm_output(y, B * T, D) if fm else _same(y, h)
    if ids.dtype != torch.int64 or ids.device != h.device or not ids.is_contiguous():
        raise ValueError("ids must be contiguous int64 on the device")
    if positions is not None and (lengths is None or positions.shape != (B, T) or positions.dtype != torch.int64
                                  or lengths.shape != (B,) or lengths.dtype != torch.int64):
        raise ValueError("positions (B, T) and lengths (B,) must be int64")
    check(_lib.lib().wptv_embed_rms_norm(ptr(ids), ptr(table), V, ptr(weight), ptr(_rows(h, "h")), ptr(_rows(y, "y")),
                                         y_blocks, B * T, D, _lib.dtype_code(h.dtype), float(eps), ptr(lengths),
                                         ptr(positions), T, _lib.stream(h.device)), "embed_rms_norm")
    return y


def add_rms_norm(h, delta, weight, y, eps=EPS):
    """h += delta (None: no add), then y = RMSNorm(h) * weight (FP32 math).
    h, delta, y share shape (..., D) and dtype; weight (D,) FP32."""
    _gpu(h, delta, weight, y)
    D = h.shape[-1]
    if y.shape != h.shape or (delta is not None and delta.shape != h.shape) or weight.shape != (D,):
        raise ValueError(f"h {tuple(h.shape)}, delta, y and weight ({D},) do not match")
    if weight.dtype != torch.float32 or (delta is not None and delta.dtype != h.dtype) or y.dtype != h.dtype:
        raise ValueError("h, delta and y share a dtype; weight is float32")
    check(_lib.lib().wptv_add_rms_norm(ptr(_rows(h, "h")), ptr(None if delta is None else _rows(delta, "delta")),
                                       ptr(weight), ptr(_rows(y, "y")), h.numel() // D, D, _lib.dtype_code(h.dtype),
                                       float(eps), _lib.stream(h.device)), "add_rms_norm")
    return y


def qkv_post(qkv, q_norm, k_norm, table, start, counts, heads, eps=EPS):
    """qkv (B, T, (H + 2) c) -> q (B, T, H, c) = q_norm per head; the entries
    [k_norm(k), v] of row b's first counts[b] tokens written into table
    (B, capacity, 2c) at start[b] + t."""
    _gpu(qkv, table)
    B, T, width = qkv.shape
    c = table.shape[-1] // 2
    if width != (heads + 2) * c or qkv.stride(-1) != 1 or qkv.stride(0) != T * qkv.stride(1):
        raise ValueError(f"qkv must be (B, T, (H + 2) c) with rows one after another; got {tuple(qkv.shape)}")
    if table.dtype != qkv.dtype or table.stride(-1) != 1 or table.shape[0] != B:
        raise ValueError("the table must be (B, capacity, 2c) in qkv's dtype, rows contiguous")
    q = torch.empty(B, T, heads, c, dtype=qkv.dtype, device=qkv.device)
    check(_lib.lib().wptv_qkv_post(ptr(qkv), qkv.stride(1), ptr(q_norm), ptr(k_norm), ptr(q), ptr(table),
                                   table.stride(0), table.stride(1), table.shape[1], ptr(start), ptr(counts), B, T,
                                   heads, c, _lib.dtype_code(qkv.dtype), float(eps), _lib.stream(qkv.device)),
          "qkv_post")
    return q


def qkv_post_parts(parts, q_norm, k_norm, table, start, counts, heads, T, eps=EPS):
    """qkv_post with the projection as FP32 split-K parts (S, B*T, (H + 2) c)
    (linear_parts' output), summed and rounded to the table's dtype first."""
    _gpu(parts, table)
    S, rows, width = parts.shape
    B = table.shape[0]
    c = table.shape[-1] // 2
    if rows != B * T or width != (heads + 2) * c or parts.dtype != torch.float32 or not parts.is_contiguous():
        raise ValueError(f"parts must be contiguous FP32 (S, B*T={B * T}, (H + 2) c={(heads + 2) * c}); "
                         f"got {tuple(parts.shape)}")
    if table.stride(-1) != 1:
        raise ValueError("the table must be (B, capacity, 2c) with contiguous rows")
    q = torch.empty(B, T, heads, c, dtype=table.dtype, device=table.device)
    check(_lib.lib().wptv_qkv_post_parts(ptr(parts), S, ptr(q_norm), ptr(k_norm), ptr(q), ptr(table),
                                         table.stride(0), table.stride(1), table.shape[1], ptr(start), ptr(counts), B,
                                         T, heads, c, _lib.dtype_code(table.dtype), float(eps),
                                         _lib.stream(table.device)), "qkv_post_parts")
    return q


def rope_divisors(dims=64, base=10000.0, device="cpu"):
    """The rotary encoding's divisors base^(2i / dims), i < dims / 2, computed
    in FP32 on the CPU as the reference's rotate computes them
    (attention.py:63-64), so that the kernel divides the same numbers."""
    pairs = torch.arange(dims // 2, dtype=torch.float32)
    return (base ** (2 * pairs / dims)).to(device)


_DIVISORS = {}  # (dims, base, device) -> rope_divisors


def window_qkv_post(proj, q_norm, k_norm, ring, start, counts, heads, rope_dims=64, rope_base=10000.0, eps=EPS):
    """A window layer after its projection: proj (B, T, >= (H + 2) c) holds
    q, k, v first (the gate may follow in the same rows) -> q (B, T, H, c) =
    rotate(q_norm(q)) at positions start[b] + t; the entries
    [rotate(k_norm(k)), v] of row b's first counts[b] tokens written into the
    ring (B, R, 2c) (R a power of 2) at row (start[b] + t) mod R
    (attention.py:113-135, rotate :59-71)."""
    _gpu(proj, ring)
    key = (int(rope_dims), float(rope_base), proj.device)
    div = _DIVISORS.get(key)
    if div is None:  # made once per setting and device, outside any graph capture
        div = _DIVISORS[key] = rope_divisors(rope_dims, rope_base, proj.device)
    B, T, width = proj.shape
    c = ring.shape[-1] // 2
    if width < (heads + 2) * c or proj.stride(-1) != 1 or proj.stride(0) != T * proj.stride(1):
        raise ValueError(f"proj must be (B, T, >= (H + 2) c) with rows one after another; got {tuple(proj.shape)}")
    if ring.dtype != proj.dtype or ring.stride(-1) != 1 or ring.shape[0] != B:
        raise ValueError("the ring must be (B, R, 2c) in proj's dtype, rows contiguous")
    q = torch.empty(B, T, heads, c, dtype=proj.dtype, device=proj.device)
    check(_lib.lib().wptv_window_qkv_post(ptr(proj), proj.stride(1), ptr(q_norm), ptr(k_norm), ptr(q), ptr(ring),
                                          ring.stride(0), ring.stride(1), ring.shape[1], ptr(start), ptr(counts), B,
                                          T, heads, c, int(rope_dims), ptr(div), _lib.dtype_code(proj.dtype),
                                          float(eps), _lib.stream(proj.device)), "window_qkv_post")
    return q


def heads_rms_norm(x, weight, heads, eps=EPS, positions=None, divisors=None):
    """x (B, T, >= H*c) (rows one after another) -> (B, T, H, c): RMSNorm of
    each head of the first H*c columns, times weight (c,) FP32.  With
    positions (B, T) int64 and divisors (rope_dims / 2,) FP32 (rope_divisors),
    each head's last rope_dims values then turned by the row's position, as
    the reference's rotate (attention.py:59-71, 130-136)."""
    _gpu(x, weight)
    B, T, width = x.shape
    c = weight.shape[0]
    if width < heads * c or x.stride(-1) != 1 or x.stride(0) != T * x.stride(1):
        raise ValueError(f"x must be (B, T, >= H*c) with rows one after another; got {tuple(x.shape)}")
    out = torch.empty(B, T, heads, c, dtype=x.dtype, device=x.device)
    if positions is None:
        check(_lib.lib().wptv_heads_rms_norm(ptr(x), x.stride(1), ptr(weight), ptr(out), B * T, heads, c,
                                             _lib.dtype_code(x.dtype), float(eps), _lib.stream(x.device)),
              "heads_rms_norm")
        return out
    _gpu(positions, divisors)
    if positions.shape != (B, T) or positions.dtype != torch.int64 or divisors.dtype != torch.float32:
        raise ValueError(f"positions must be int64 ({B}, {T}) and divisors FP32; got {tuple(positions.shape)} "
                         f"{positions.dtype}, {divisors.dtype}")
    positions = positions.contiguous()
    check(_lib.lib().wptv_heads_rms_norm_rope(ptr(x), x.stride(1), ptr(weight), ptr(out), B * T, heads, c,
                                              _lib.dtype_code(x.dtype), float(eps), ptr(positions),
                                              2 * divisors.shape[0], ptr(divisors), _lib.stream(x.device)),
          "heads_rms_norm_rope")
    return out


def swiglu(gate_up):
    """silu(gate) * up of gate_up (..., 2F): (..., F)."""
    _gpu(gate_up)
    F = gate_up.shape[-1] // 2
    out = torch.empty(*gate_up.shape[:-1], F, dtype=gate_up.dtype, device=gate_up.device)
    check(_lib.lib().wptv_swiglu(ptr(_rows(gate_up, "gate_up")), ptr(out), gate_up.numel() // (2 * F), F,
                                 _lib.dtype_code(gate_up.dtype), _lib.stream(gate_up.device)), "swiglu")
    return out


def wide_tiles(M, N, K):
    """Whether wptv_gemm runs an unsplit product of M rows on its 256 x 256
    tiles (gemm_wide.hip): above 320 rows, N a multiple of 256, K of 32."""
    return M >= WIDE_MIN_ROWS and N % 256 == 0 and K % 32 == 0


def linear(x, w, out_dtype=None, splits=0):
    """x (..., K) . w (N, K)^T on the matrix cores (the projections' and the
    lm_head's nn.Linear under bf16 autocast): bf16 operands, FP32
    accumulation; out_dtype bfloat16 (default) or float32 (the bf16-rounded
    product as FP32).  Up to 512 rows on the skinny products (N and K
    multiples of 64); with splits 0, above 320 rows, any number of rows on the
    wide tiles (N a multiple of 256, K of 32)."""
    _gpu(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError(f"linear takes bf16 operands; got {x.dtype} and {w.dtype}")
    K = x.shape[-1]
    N = w.shape[0]
    if w.dim() != 2 or w.shape[1] != K or w.stride(1) != 1:
        raise ValueError(f"w must be (N, K={K}) with contiguous rows; got {tuple(w.shape)}")
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    out_dtype = torch.bfloat16 if out_dtype is None else out_dtype
    code = _lib.dtype_code(out_dtype)
    library = _lib.lib()
    parts = _lib.ctypes.c_int(int(splits))
    size = _lib.ctypes.c_size_t(0)
    if not (splits == 0 and wide_tiles(M, N, K)):  # the wide tiles need no split count and no workspace
        check(library.wptv_gemm_workspace(M, N, K, _lib.ctypes.byref(parts), _lib.ctypes.byref(size)), "gemm")
    workspace = torch.empty(size.value, dtype=torch.uint8, device=x.device) if size.value else None
    out = torch.empty(M, N, dtype=out_dtype, device=x.device)
    check(library.wptv_gemm(ptr(x2), x2.stride(0), ptr(w), w.stride(0), M, N, K, ptr(out), out.stride(0), code,
                            parts.value, ptr(workspace), size.value, _lib.stream(x.device)), "gemm")
    return out.reshape(*x.shape[:-1], N)


def interleave_gate_up(gate_up):
    """(2F, K) gate rows then up rows -> the tile-interleaved order
    linear_swiglu reads: for each 32 features, their 32 gate rows then their
    32 up rows (F a multiple of 32)."""
    F2, K = gate_up.shape
    F = F2 // 2
    if F2 % 2 or F % 32:
        raise ValueError(f"gate_up must hold 2F rows, F a multiple of 32; got {F2}")
    gate, up = gate_up[:F].view(F // 32, 32, K), gate_up[F:].view(F // 32, 32, K)
    return torch.cat([gate, up], 1).reshape(F2, K).contiguous()


def linear_swiglu(x, w_interleaved):
    """silu(x . gate^T) * (x . up^T) of x (..., K) and the interleaved gate/up
    weight (2F, K) (interleave_gate_up), on the matrix cores with SwiGLU in
    the product's epilogue: bf16 (..., F).  At most 512 rows."""
    _gpu(x, w_interleaved)
    if x.dtype != torch.bfloat16 or w_interleaved.dtype != torch.bfloat16:
        raise ValueError(f"linear_swiglu takes bf16 operands; got {x.dtype} and {w_interleaved.dtype}")
    K = x.shape[-1]
    N = w_interleaved.shape[0]
    if w_interleaved.dim() != 2 or w_interleaved.shape[1] != K or w_interleaved.stride(1) != 1:
        raise ValueError(f"w must be (2F, K={K}) with contiguous rows; got {tuple(w_interleaved.shape)}")
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    out = torch.empty(M, N // 2, dtype=torch.bfloat16, device=x.device)
    check(_lib.lib().wptv_gemm_swiglu(ptr(x2), x2.stride(0), ptr(w_interleaved), w_interleaved.stride(0), M, N, K,
                                      ptr(out), out.stride(0), _lib.stream(x.device)), "gemm_swiglu")
    return out.reshape(*x.shape[:-1], N // 2)


def linear_parts(x, w, splits=0, max_splits=8):
    """The split-K parts of x (..., K) . w (N, K)^T: FP32 (S, rows, N) whose
    sum over S is the product (wptv_gemm_parts), for a consumer that sums them
    (add_rms_norm_parts, which takes up to 8).  splits 0: the library's
    choice, at most max_splits."""
    _gpu(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError(f"linear_parts takes bf16 operands; got {x.dtype} and {w.dtype}")
    K = x.shape[-1]
    N = w.shape[0]
    if w.dim() != 2 or w.shape[1] != K or w.stride(1) != 1:
        raise ValueError(f"w must be (N, K={K}) with contiguous rows; got {tuple(w.shape)}")
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    library = _lib.lib()
    parts = _lib.ctypes.c_int(int(splits))
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_gemm_workspace(M, N, K, _lib.ctypes.byref(parts), _lib.ctypes.byref(size)), "gemm_parts")
    if parts.value > max_splits:
        parts = _lib.ctypes.c_int(int(max_splits))
        check(library.wptv_gemm_workspace(M, N, K, _lib.ctypes.byref(parts), _lib.ctypes.byref(size)), "gemm_parts")
    out = torch.empty(parts.value, M, N, dtype=torch.float32, device=x.device)
    check(library.wptv_gemm_parts(ptr(x2), x2.stride(0), ptr(w), w.stride(0), M, N, K, parts.value, ptr(out),
                                  out.numel() * 4, _lib.stream(x.device)), "gemm_parts")
    return out


def add_rms_norm_parts(h, parts, weight, y, eps=EPS, fm=False):
    """add_rms_norm with delta = parts.sum(0) (FP32 (S, rows, D), S <= 8),
    rounded to h's dtype before the residual add.  fm: y is a flat
    fragment-major operand of the rows (fm_empty), not h's shape."""
    _gpu(h, parts, weight, y)
    D = h.shape[-1]
    M = h.numel() // D
    if parts.dim() != 3 or parts.shape[1:] != (M, D) or parts.dtype != torch.float32 or not parts.is_contiguous():
        raise ValueError(f"parts must be contiguous FP32 (S, {M}, {D}); got {tuple(parts.shape)} {parts.dtype}")
    if y.dtype != h.dtype or weight.shape != (D,) or weight.dtype != torch.float32:
        raise ValueError("h and y share a dtype; weight is float32 (D,)")
    y_blocks = _fm_output(y, M, D) if fm else _same(y, h)
    check(_lib.lib().wptv_add_rms_norm_parts(ptr(_rows(h, "h")), ptr(parts), parts.shape[0], ptr(weight),
                                             ptr(_rows(y, "y")), y_blocks, M, D, _lib.dtype_code(h.dtype),
                                             float(eps), _lib.stream(h.device)), "add_rms_norm_parts")
    return y


# ---- fragment-major operands (include/wptv.h) and the products that read them ----

FM_MAX_ROWS = 320  # rows the fm products take (up to 160, or 289 to 320)


def _same(y, h):
    if y.shape != h.shape:
        raise ValueError(f"y must have h's shape {tuple(h.shape)}; got {tuple(y.shape)}")
    return 0


def _fm_output(y, rows, width):
    """The row blocks of y, a flat fm operand of rows x width."""
    blocks = _lib.fm_row_blocks(rows)
    if y.dtype != torch.bfloat16 or y.dim() != 1 or y.numel() < blocks * 16 * width or width % 32:
        raise ValueError(f"an fm operand of {rows} x {width} is a flat bf16 tensor of {blocks * 16 * width} "
                         f"elements (width a multiple of 32); got {tuple(y.shape)} {y.dtype}")
    return blocks


def fm_empty(rows, width, device, dtype=torch.bfloat16):
    """An uninitialised flat fm operand of rows x width (padding rows included)."""
    return torch.empty(_lib.fm_row_blocks(rows) * 16 * width, dtype=dtype, device=device)


def fm_pack(a, row_blocks=None):
    """a (R, K) bf16 in the fm layout, flat, with row_blocks 16-row blocks
    (default: fm_row_blocks(R)); padding rows zero (wptv_fm_pack)."""
    _gpu(a)
    if a.dtype != torch.bfloat16 or a.dim() != 2 or a.stride(1) != 1:
        raise ValueError(f"fm_pack takes a bf16 (R, K) matrix with contiguous rows; got {tuple(a.shape)} {a.dtype}")
    R, K = a.shape
    blocks = _lib.fm_row_blocks(R) if row_blocks is None else int(row_blocks)
    out = torch.empty(blocks * 16 * K, dtype=a.dtype, device=a.device)
    check(_lib.lib().wptv_fm_pack(ptr(a), a.stride(0), R, K, blocks, ptr(out), _lib.stream(a.device)), "fm_pack")
    return out


def fm_unpack(packed, rows, width):
    """The (rows, width) row-major matrix of a flat fm operand (torch
    reshapes: element 8 l + e of block (ks, rb) is row 16 rb + l % 16,
    column 32 ks + 8 (l // 16) + e)."""
    blocks = packed.numel() // (16 * width)
    a = packed[: blocks * 16 * width].view(width // 32, blocks, 4, 16, 8)  # ks, rb, g, j, e
    return a.permute(1, 3, 0, 2, 4).reshape(blocks * 16, width)[:rows]


class FmWeight:
    """A weight (N, K) packed once in the fm layout (N / 16 row blocks)."""

    def __init__(self, w):
        self.shape = tuple(w.shape)
        self.data = fm_pack(w.contiguous(), w.shape[0] // 16)


def fm_plan(M, N, K, swiglu=False):
    """(parts, parts bytes) of an fm product, or None where no kernel form
    takes the shape."""
    if not 0 < M <= FM_MAX_ROWS:
        return None
    parts = _lib.ctypes.c_int(1 if swiglu else 0)
    size = _lib.ctypes.c_size_t(0)
    status = _lib.lib().wptv_gemm_fm_plan(M, N, K, int(swiglu), _lib.ctypes.byref(parts), _lib.ctypes.byref(size))
    return (parts.value, size.value) if status == 0 else None


def linear_fm_parts(x_fm, rows, w, splits=0):
    """The split-K parts (S, rows, N) FP32 of x . w^T, x a flat fm operand of
    rows x K, w an FmWeight (N, K) (wptv_gemm_fm_parts)."""
    _gpu(x_fm, w.data)
    N, K = w.shape
    _fm_output(x_fm, rows, K)
    library = _lib.lib()
    parts = _lib.ctypes.c_int(int(splits))
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_gemm_fm_plan(rows, N, K, 0, _lib.ctypes.byref(parts), _lib.ctypes.byref(size)), "gemm_fm")
    out = torch.empty(parts.value, rows, N, dtype=torch.float32, device=x_fm.device)
    check(library.wptv_gemm_fm_parts(ptr(x_fm), ptr(w.data), rows, N, K, parts.value, ptr(out), out.numel() * 4,
                                     _lib.stream(x_fm.device)), "gemm_fm_parts")
    return out


def linear_fm_wide(x_fm, rows, w, out_dtype=torch.bfloat16):
    """x . w^T on the 256 x 256 tiles: x a flat fm operand of rows x K, w an
    FmWeight (N, K), N a multiple of 256 (wptv_gemm_fm_wide; the lm_head of a
    reading of many rows).  Returns (rows, N) bf16, or FP32 holding the
    bf16-rounded product."""
    _gpu(x_fm, w.data)
    N, K = w.shape
    _fm_output(x_fm, rows, K)
    blocks = x_fm.numel() // (16 * K)  # every row block the operand holds
    out = torch.empty(rows, N, dtype=out_dtype, device=x_fm.device)
    check(_lib.lib().wptv_gemm_fm_wide(ptr(x_fm), blocks, ptr(w.data), rows, N, K, ptr(out), out.stride(0),
                                       _lib.dtype_code(out_dtype), _lib.stream(x_fm.device)), "gemm_fm_wide")
    return out


def head_argmax_fm_wide(x_fm, rows, w):
    """Each row's first maximal index of the bf16-rounded product x . w^T (the
    greedy decisions' argmax of an lm_head's logits), without storing the
    product: (rows,) int32, in torch.argmax's order (a NaN the largest value)
    (wptv_gemm_fm_wide_argmax).
    x a flat fm operand of rows x K, w an FmWeight (N, K), N a multiple of 256."""
    _gpu(x_fm, w.data)
    N, K = w.shape
    _fm_output(x_fm, rows, K)
    blocks = x_fm.numel() // (16 * K)
    library = _lib.lib()
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_gemm_fm_wide_argmax_workspace(rows, N, _lib.ctypes.byref(size)), "gemm_fm_wide_argmax")
    workspace = torch.empty(size.value, dtype=torch.uint8, device=x_fm.device)
    best = torch.empty(rows, dtype=torch.int32, device=x_fm.device)
    check(library.wptv_gemm_fm_wide_argmax(ptr(x_fm), blocks, ptr(w.data), rows, N, K, ptr(best), ptr(workspace),
                                           size.value, _lib.stream(x_fm.device)), "gemm_fm_wide_argmax")
    return best


def linear_fm_swiglu(x_fm, rows, w):
    """silu(gate) * up of x (a flat fm operand of rows x K) and the gate/up
    FmWeight packed from interleave_gate_up's order: a flat fm operand of
    rows x N / 2, the down product's X (wptv_gemm_fm_swiglu)."""
    _gpu(x_fm, w.data)
    N, K = w.shape
    _fm_output(x_fm, rows, K)
    out = fm_empty(rows, N // 2, x_fm.device)
    check(_lib.lib().wptv_gemm_fm_swiglu(ptr(x_fm), ptr(w.data), rows, N, K, ptr(out), _lib.stream(x_fm.device)),
          "gemm_fm_swiglu")
    return out
