"""An MQA decoder behind the reference's generation protocol (new_cache /
extend / undo, packages/wpt-model/src/wpt_model/model.py:451-483), running
its verify-step hot path on libwptv's HIP kernels.

Each layer is the reference's exact layer (ExactAttention, attention.py:
157-188: q = q_norm(q(x)) per head, the entries [k_norm(k(x)), v(x)] of the
new tokens appended to the cache, exact attention of every query over the
rows up to its position, the output projection) in a pre-norm residual
block, then a SwiGLU feed-forward block; a final norm and the head give
FP32 scores (model.py:471).  One key/value head is shared by every query
head (MQA).  RMSNorm's eps is the reference's (layers.py:9).  A layer may
instead be the reference's window layer (WindowAttention, attention.py:
109-151): rotary encoding of the normed queries and key, a window of the last
`window` tokens with a sink per head, and the output gated by sigmoid(gate(x)),
or the reference's sparse layer (SparseAttention, attention.py:191-216): the
normed queries attend to the rows the exact layer before it chose for each
query (its top_k rows outside the last `window`, by the largest
max_h log-softmax weight) and to the last `window` rows of that layer's table,
with a sink per head and the same output gate.  An exact layer followed by a
sparse layer makes that choice (model.py:134-135); layer_kinds gives the
reference's layout of the three kinds (config.py:17-23).

On the GPU:
    the input       wptv_embed_rms_norm: the embedding rows, the first norm
                    and each token's position in one pass
    KV append       wptv_qkv_post: q/k norms, and the new entries written at
                    each row's own length (no host sync)
    norms, SwiGLU   wptv_add_rms_norm (residual add + RMSNorm), wptv_swiglu
    the lengths     wptv_cache_lengths after the reading and after an undo
    verify attention wptv_verify_attention, reading only the rows the query
                    positions reach in the cache's table
    projections     the matrix products of the dtype on MFMA: at up to 160
                    bf16 rows the fragment-major products (wptv_gemm_fm_*:
                    weights packed once, X written in that layout by the
                    norms, the attention and the SwiGLU epilogue) for the
                    exact layers' q/k/v and output and every feed-forward
                    block; wptv_gemm's split-K parts otherwise up to
                    SPLIT_K_ROWS bf16 rows (summed by qkv_post and the
                    residual add + norm), the gate/up product with SwiGLU in
                    its epilogue (wptv_gemm_swiglu) at up to 512 bf16 rows;
                    the lm_head on wptv_gemm (the skinny products up to 320
                    rows, the 256 x 256 tiles above); hipBLASLt only for a
                    prefill's wider layer products
    window layers   wptv_window_qkv_post (norms, rotary encoding, the ring
                    append), wptv_window_attention over the cache's ring with
                    the sink and the output gate fused
    sparse layers   the exact layer's lse (wptv_verify_attention) and choice
                    (wptv_exact_choice), wptv_heads_rms_norm for the queries,
                    wptv_sparse_attention over the exact layer's table with
                    the sink and the output gate fused
    sampling        wpt_amd.sampling (wptv_accept), called by the Writer
The decoder keeps no state between calls but the cache; a step of fixed
shape can be captured in a HIP graph (wpt_amd.step).
"""

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import kernels, layers
from .cache import Cache

EPS = 1e-6
# Rows up to which the projections run as the build's split-K products: at
# 160 rows (batch 32, k = 4) the step takes 2.53 ms with them against 2.81 ms
# with hipBLASLt; at 320 rows (batch 64) the two tie (3.19 vs 3.16 ms).
SPLIT_K_ROWS = 320


WINDOW, EXACT, SPARSE = "window", "exact", "sparse"


def layer_kinds(window_layers, sparse_groups, sparse_layers):
    """The reference's layout of layer kinds (config.py:17-23): window layers
    around one exact layer, then groups of one exact layer and the sparse
    layers that read it."""
    first = (WINDOW,) * window_layers + (EXACT,) + (WINDOW,) * window_layers
    return first + ((EXACT,) + (SPARSE,) * sparse_layers) * sparse_groups


@dataclass(frozen=True)
class DecoderConfig:
    layers: int
    d_model: int
    heads: int
    head_dim: int
    ffn: int
    vocab: int
    kinds: tuple = ()          # "exact", "window" or "sparse" per layer; () = every layer exact
    window: int = 128          # WINDOW, attention.py:53
    rope_dims: int = 64        # ROPE_DIMS, attention.py:55
    rope_base: float = 10000.0  # ROPE_BASE, attention.py:56
    top_k: int = 1024          # TOP_K, attention.py:54: rows an exact layer chooses for the sparse layers

    def __post_init__(self):
        if self.kinds:
            if len(self.kinds) != self.layers or set(self.kinds) - {WINDOW, EXACT, SPARSE}:
                raise ValueError(f"kinds must name one of {WINDOW!r}, {EXACT!r}, {SPARSE!r} for each of the "
                                 f"{self.layers} layers; got {self.kinds}")
            for i, kind in enumerate(self.kinds):
                if kind == SPARSE and (i == 0 or self.kinds[i - 1] == WINDOW):
                    raise ValueError(f"sparse layer {i} follows no exact layer or sparse layer: it has no "
                                     "choice of rows to read")

    @property
    def qkv_width(self):
        return self.heads * self.head_dim + 2 * self.head_dim

    def kind(self, i):
        return self.kinds[i] if self.kinds else EXACT

    @property
    def windows(self):
        """The window layers' indices."""
        return tuple(i for i in range(self.layers) if self.kind(i) == WINDOW)

    @property
    def sparse(self):
        """The sparse layers' indices."""
        return tuple(i for i in range(self.layers) if self.kind(i) == SPARSE)

    def chooses(self, i):
        """Whether exact layer i chooses rows: a sparse layer follows it."""
        return self.kind(i) == EXACT and i + 1 < self.layers and self.kind(i + 1) == SPARSE


# The decoders of the verify-step workloads.
PLUMBING = DecoderConfig(layers=4, d_model=256, heads=4, head_dim=64, ffn=704, vocab=8192)
LARGE = DecoderConfig(layers=24, d_model=2048, heads=16, head_dim=128, ffn=5632, vocab=32768)


def random_weights(config, seed=0, std=0.02, dtype=torch.float32, device="cpu"):
    """Random-init weights: every matrix ~ N(0, std) drawn from one seeded
    generator on `device` in a fixed order, every norm weight 1."""
    generator = torch.Generator(device=device).manual_seed(seed)
    D, H, c, Fw, V = config.d_model, config.heads, config.head_dim, config.ffn, config.vocab

    def normal(*shape):
        return (torch.randn(*shape, generator=generator, device=device) * std).to(dtype)

    def ones(n):
        return torch.ones(n, dtype=torch.float32, device=device)

    weights = {"embedding": normal(V, D)}
    for i in range(config.layers):
        weights[f"layers.{i}.attn_norm"] = ones(D)
        if config.kind(i) == SPARSE:  # queries only: the keys and values are the exact layer's
            weights[f"layers.{i}.q"] = normal(H * c, D)
        else:
            weights[f"layers.{i}.qkv"] = normal(config.qkv_width, D)
        weights[f"layers.{i}.q_norm"] = ones(c)
        if config.kind(i) != SPARSE:
            weights[f"layers.{i}.k_norm"] = ones(c)
        weights[f"layers.{i}.out"] = normal(D, H * c)
        weights[f"layers.{i}.ffn_norm"] = ones(D)
        weights[f"layers.{i}.gate_up"] = normal(2 * Fw, D)
        weights[f"layers.{i}.down"] = normal(D, Fw)
        if config.kind(i) in (WINDOW, SPARSE):
            weights[f"layers.{i}.gate"] = normal(H * c, D)
            # the reference starts its sinks at 0; drawn here so that they matter
            weights[f"layers.{i}.sink"] = torch.randn(H, generator=generator, device=device)
    weights["final_norm"] = ones(D)
    weights["head"] = normal(V, D)
    return weights


class MQADecoder:
    """config: DecoderConfig; weights: random_weights' names; dtype: the
    compute dtype (float32 or bfloat16), on a GPU."""

    def __init__(self, config, weights, dtype=torch.bfloat16, device="cuda"):
        self.config, self.dtype = config, dtype
        self.device = torch.device(device)
        self._widths = {}
        if self.device.type != "cuda":
            raise kernels.KernelUnavailable(f"the decoder's verify step runs on a GPU, not {self.device}")
        self.w = {}
        for name, value in weights.items():
            keep_fp32 = name.endswith("norm") or name.endswith("sink")
            self.w[name] = value.to(device=self.device, dtype=torch.float32 if keep_fp32 else dtype).contiguous()
        for i in config.windows:  # one projection for q, k, v and the gate
            self.w[f"layers.{i}.qkvg"] = torch.cat([self.w[f"layers.{i}.qkv"], self.w[f"layers.{i}.gate"]]).contiguous()
        for i in config.sparse:  # one projection for q and the gate
            self.w[f"layers.{i}.qg"] = torch.cat([self.w[f"layers.{i}.q"], self.w[f"layers.{i}.gate"]]).contiguous()
        if dtype == torch.bfloat16:  # the gate/up rows in the order the fused SwiGLU product reads, kept instead
            for i in range(config.layers):
                self.w[f"layers.{i}.gate_up_tiles"] = layers.interleave_gate_up(self.w.pop(f"layers.{i}.gate_up"))
        # the fm products' weights, packed once (beside the row-major ones that wider readings use)
        self.fm = {}
        if dtype == torch.bfloat16:
            for i in range(config.layers):
                names = ["gate_up_tiles", "down"] + (["qkv", "out"] if config.kind(i) == EXACT else [])
                for name in names:
                    key = f"layers.{i}.{name}"
                    self.fm[key] = layers.FmWeight(self.w[key])
        self._fm_rows = {}

    def parameters(self):
        return iter(self.w.values())

    def new_cache(self, rows, routes=False, capacity=256, widest=129):
        """An empty cache of `rows` rows (the reference's WPT.new_cache); its
        window layers' rings hold readings of up to `widest` tokens (wider
        ones are read in pieces)."""
        if routes:
            raise NotImplementedError("this decoder has no routed experts to record")
        c = self.config.head_dim
        ring = 1 << max(0, (self.config.window - 1 + widest - 1).bit_length())
        return Cache(rows, self.config.layers, 2 * c, self.dtype, self.device, capacity, self.config.windows, ring,
                     self.config.sparse)

    def widest(self, cache):
        """The most tokens one reading of the cache takes (its rings' size)."""
        ring = cache.ring_rows
        return None if ring is None else ring - self.config.window + 1

    def fm_rows(self, rows):
        """Whether a reading of `rows` rows runs the fm products (bf16, up to
        160 rows or 289 to 320, every layer's shapes taken by a kernel form)."""
        ok = self._fm_rows.get(rows)
        if ok is None:
            ok = self.dtype == torch.bfloat16 and all(
                layers.fm_plan(rows, w.shape[0], w.shape[1], swiglu=name.endswith("gate_up_tiles")) is not None
                for name, w in self.fm.items())
            self._fm_rows[rows] = ok
        return ok

    def _attn_input_fm(self, i, fm):
        """Whether layer i's attention block reads its input x in the fm layout."""
        return fm and i < self.config.layers and self.config.kind(i) == EXACT

    def _layer(self, i, h, x, cache, positions, counts, next_norm, handoff, xf=None):
        """One layer on the residual stream h (B, T, D), x = RMSNorm(h) with the
        layer's attention norm; leaves h updated and x = RMSNorm(h) with
        next_norm (the next layer's attention norm, or the final norm).
        handoff: what the last exact layer gave the sparse layers; returns
        the handoff for the next layer.  xf: a flat fm operand of the rows
        when the reading runs the fm products: the norms write x there
        instead of into x when the product that reads it is an fm one (an
        exact layer's q/k/v, every feed-forward block)."""
        w = self.w
        B, T, _ = h.shape
        kind = self.config.kind(i)
        fm = xf is not None
        x_in = xf if self._attn_input_fm(i, fm) else x
        if kind == WINDOW:
            self._window_attention(i, h, x_in, cache, positions, counts, xf)
        elif kind == SPARSE:
            self._sparse_attention(i, h, x_in, positions, handoff, xf)
        else:
            handoff = self._exact_attention(i, h, x_in, cache, positions, counts, xf)
        if fm:
            act = layers.linear_fm_swiglu(xf, B * T, self.fm[f"layers.{i}.gate_up_tiles"])
            nxt = self._attn_input_fm(i + 1, fm)
            layers.add_rms_norm_parts(h, layers.linear_fm_parts(act, B * T, self.fm[f"layers.{i}.down"]), next_norm,
                                      xf if nxt else x, fm=nxt)
            return handoff
        if x.dtype != torch.bfloat16:
            act = layers.swiglu(F.linear(x, w[f"layers.{i}.gate_up"]))
        elif B * T <= layers.LINEAR_MAX_ROWS:
            act = layers.linear_swiglu(x, w[f"layers.{i}.gate_up_tiles"])  # SwiGLU in the product's epilogue
        else:  # wider readings (a prefill): the product, then SwiGLU of its tile-interleaved halves
            gu = F.linear(x, w[f"layers.{i}.gate_up_tiles"]).unflatten(-1, (-1, 2, 32))
            act = (F.silu(gu[..., 0, :].float()) * gu[..., 1, :].float()).flatten(-2).to(x.dtype)
        down = w[f"layers.{i}.down"]
        if x.dtype == torch.bfloat16 and B * T <= SPLIT_K_ROWS:
            layers.add_rms_norm_parts(h, layers.linear_parts(act, down), next_norm, x)
        else:
            layers.add_rms_norm(h, F.linear(act, down), next_norm, x)
        return handoff

    @staticmethod
    def _linear(x, w):
        """x . w^T in x's dtype: the build's product for bf16 at up to
        LINEAR_MAX_ROWS rows, torch's otherwise (FP32, or a wide prefill)."""
        if x.dtype == torch.bfloat16 and x.numel() // x.shape[-1] <= layers.LINEAR_MAX_ROWS:
            return layers.linear(x, w)
        return F.linear(x, w)

    def _attention_out(self, i, h, x, o, xf=None):
        """h += out(o), x = RMSNorm(h) with the feed-forward norm (into xf,
        the fm operand, when given).  o (B, T, H, c), or a flat fm operand of
        the B T rows."""
        if xf is not None:
            B, T, D = h.shape
            rows = B * T
            if o.dim() == 1:
                parts = layers.linear_fm_parts(o, rows, self.fm[f"layers.{i}.out"])
            else:
                parts = layers.linear_parts(o.reshape(rows, -1), self.w[f"layers.{i}.out"])
            layers.add_rms_norm_parts(h, parts, self.w[f"layers.{i}.ffn_norm"], xf, fm=True)
            return
        B, T, H, c = o.shape
        out = self.w[f"layers.{i}.out"]
        if x.dtype == torch.bfloat16 and B * T <= SPLIT_K_ROWS:
            layers.add_rms_norm_parts(h, layers.linear_parts(o.reshape(B, T, H * c), out),
                                      self.w[f"layers.{i}.ffn_norm"], x)
        else:
            layers.add_rms_norm(h, F.linear(o.reshape(B, T, H * c), out), self.w[f"layers.{i}.ffn_norm"], x)

    def _window_attention(self, i, h, x, cache, positions, counts, xf=None):
        """A window layer's attention block: h += out(o * sigmoid(gate(x))),
        x = RMSNorm(h) with the feed-forward norm."""
        w, cfg = self.w, self.config
        B, T, _ = h.shape
        H, c = cfg.heads, cfg.head_dim
        ring = cache.tables[i]
        proj = self._linear(x, w[f"layers.{i}.qkvg"])  # (B, T, (2H + 2) c): q, k, v, gate
        q = layers.window_qkv_post(proj, w[f"layers.{i}.q_norm"], w[f"layers.{i}.k_norm"], ring, cache.lengths,
                                   counts, H, cfg.rope_dims, cfg.rope_base)
        o = kernels.ring_attention(q, ring, positions, c ** -0.5, cfg.window, w[f"layers.{i}.sink"],
                                   gate=proj[..., (H + 2) * c:])
        self._attention_out(i, h, x, o, xf)

    def _sparse_attention(self, i, h, x, positions, handoff, xf=None):
        """A sparse layer's attention block over the exact layer's table and
        choice (handoff = (keys, values, chosen)): h += out(o * sigmoid(gate(x))),
        x = RMSNorm(h) with the feed-forward norm."""
        w, cfg = self.w, self.config
        H, c = cfg.heads, cfg.head_dim
        keys, values, chosen = handoff
        proj = self._linear(x, w[f"layers.{i}.qg"])  # (B, T, 2 H c): q, gate
        q = layers.heads_rms_norm(proj, w[f"layers.{i}.q_norm"], H)
        o = kernels.sparse_attention(q, keys, values, w[f"layers.{i}.sink"], chosen, positions, c ** -0.5, cfg.window,
                                     gate=proj[..., H * c:])
        self._attention_out(i, h, x, o, xf)

    def _exact_attention(self, i, h, x, cache, positions, counts, xf=None):
        """An exact layer's attention block: h += out(o), x = RMSNorm(h) with
        the feed-forward norm.  Returns (keys, values, chosen), the sparse
        layers' handoff (chosen None when no sparse layer follows).  xf
        given: x is that fm operand, and the output goes through the fm
        products."""
        w, cfg = self.w, self.config
        B, T, _ = h.shape
        H, c = cfg.heads, cfg.head_dim
        table = cache.tables[i]
        fm = xf is not None
        # at the verify step's few bf16 rows, the projections run as the
        # build's split-K MFMA products (each weight read once), their FP32
        # parts summed by the kernel that consumes them; torch's otherwise
        few = h.dtype == torch.bfloat16 and B * T <= SPLIT_K_ROWS
        if fm:
            q = layers.qkv_post_parts(layers.linear_fm_parts(xf, B * T, self.fm[f"layers.{i}.qkv"]),
                                      w[f"layers.{i}.q_norm"], w[f"layers.{i}.k_norm"], table, cache.lengths, counts,
                                      H, T)
        elif few:
            q = layers.qkv_post_parts(layers.linear_parts(x, w[f"layers.{i}.qkv"]), w[f"layers.{i}.q_norm"],
                                      w[f"layers.{i}.k_norm"], table, cache.lengths, counts, H, T)
        else:
            qkv = F.linear(x, w[f"layers.{i}.qkv"])
            q = layers.qkv_post(qkv, w[f"layers.{i}.q_norm"], w[f"layers.{i}.k_norm"], table, cache.lengths, counts,
                                H)
        keys, values = table[..., :c], table[..., c:]
        chosen = None
        if cfg.chooses(i):  # the top_k rows outside the window by the largest max_h log-softmax weight
            o, lse = kernels.verify_attention(q, keys, values, positions, c ** -0.5, lse=True, from_positions=True,
                                              out_fm=fm)
            chosen = kernels.choose_rows(q, keys, positions, lse, c ** -0.5, cfg.top_k, cfg.window)
        else:
            o = kernels.verify_attention(q, keys, values, positions, c ** -0.5, from_positions=True, out_fm=fm)
        self._attention_out(i, h, x, o, xf)
        return keys, values, chosen

    @torch.no_grad()
    def extend(self, ids, cache, counts=None, undoable=False, features=(), logits=False):
        """Reads ids (B, n), the next tokens of the cache's B rows: the first
        counts[b] of row b (all n by default), the rest padding.  Returns
        ((B, n, V) FP32 scores, (B, n, D) final hidden states), as the
        reference's WPT.extend (model.py:456-473); with features (layer
        numbers 0 .. layers), also the residual stream entering each named
        layer (`layers` naming the final hidden states), FP32, side by side
        in the order named: (B, n, D * len(features)) (model.py:406-436).
        logits=True: the scores in the compute dtype as the head gives them,
        before the reference's .float() (the sampler reads bf16 scores as
        those exact FP32 values)."""
        features = tuple(int(n) for n in features)
        if any(not 0 <= n <= self.config.layers for n in features):
            raise ValueError(f"features name layers 0 .. {self.config.layers}; got {features}")
        if ids.device.type == "cpu" and ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self.config.vocab):
            raise IndexError(f"token ids must lie in [0, {self.config.vocab})")
        ids = ids.to(device=self.device, dtype=torch.long)
        B, T = ids.shape
        if B != cache.rows:
            raise ValueError(f"ids hold {B} rows; the cache {cache.rows}")
        if counts is None:  # every token of every row: one device tensor per width, made once and kept
            # (a captured step replays the tensor it read, so none is ever dropped)
            counts_ = self._widths.get((B, T))
            if counts_ is None:
                counts_ = self._widths[(B, T)] = torch.full((B,), T, dtype=torch.long, device=self.device)
        else:
            counts_ = torch.as_tensor(counts, dtype=torch.long).to(self.device)
        widest = self.widest(cache)
        if widest is not None and T > widest:
            if undoable:
                raise ValueError(f"an undoable reading of {T} tokens is wider than the cache's rings take ({widest})")
            # in pieces that the window layers' rings hold; every layer is causal
            pieces = []
            for start in range(0, T, widest):
                part = self.extend(ids[:, start:start + widest], cache, (counts_ - start).clamp(0, widest),
                                   features=features, logits=logits)
                pieces.append(part)
            return tuple(torch.cat([p[i] for p in pieces], 1) for i in range(len(pieces[0])))
        cache.reserve(cache.bound + T)
        D = self.config.d_model
        h = torch.empty(B, T, D, dtype=self.dtype, device=self.device)
        x = torch.empty_like(h)
        positions = torch.empty(B, T, dtype=torch.long, device=self.device)
        # the fm products' operand: x in the fragment-major layout
        xf = layers.fm_empty(B * T, D, self.device) if self.fm_rows(B * T) else None
        first_fm = self._attn_input_fm(0, xf is not None)
        # the embedding, the first norm and each token's position in one pass
        layers.embed_rms_norm(ids.contiguous(), self.w["embedding"], self.w["layers.0.attn_norm"], h,
                              xf if first_fm else x, cache.lengths, positions, fm=first_fm)
        found = {}
        handoff = None
        for i in range(self.config.layers):
            if i in features:  # the stream entering layer i (the layers update h in place)
                found[i] = h.float()
            last = i + 1 == self.config.layers
            next_norm = self.w["final_norm"] if last else self.w[f"layers.{i + 1}.attn_norm"]
            handoff = self._layer(i, h, x, cache, positions, counts_, next_norm, handoff, xf)
        if self.config.layers in features:
            found[self.config.layers] = h.float()
        head = self.w["head"]
        if x.dtype == torch.bfloat16 and (B * T <= layers.LINEAR_MAX_ROWS
                                          or layers.wide_tiles(B * T, head.shape[0], head.shape[1])):
            # the build's product (the skinny products up to 320 rows, the wide tiles
            # above); FP32 output = the bf16 product's values, the reference's .float()
            scores = layers.linear(x, head, out_dtype=torch.bfloat16 if logits else torch.float32)
        else:
            scores = F.linear(x, head)
            if not logits:
                scores = scores.float()
        cache.finish(counts_, undoable, T)
        if features:
            return scores, h, torch.cat([found[n] for n in features], -1)
        return scores, h

    @torch.no_grad()
    def undo(self, cache, kept):
        """After an undoable extend: keeps only its first kept[b] tokens of
        row b (the reference's WPT.undo, model.py:475-483); kept int64 or
        int32 (a sampler's counts), on the device or the host."""
        if not (torch.is_tensor(kept) and kept.dtype in (torch.int64, torch.int32)):
            kept = torch.as_tensor(kept, dtype=torch.long)
        cache.undo(kept.to(self.device))

    @torch.no_grad()
    def __call__(self, ids):
        """The scores (B, T, V) of each row's whole text, read in one pass."""
        ids = ids.to(self.device)
        return self.extend(ids, self.new_cache(ids.shape[0], capacity=ids.shape[1]))[0]
