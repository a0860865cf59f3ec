"""Oracle MQA decoder: the verify step's model, restated on the CPU in FP32
(test infrastructure; see oracle/__init__.py).

The decoder is built from the reference's exact layer (ExactAttention,
packages/wpt-model/src/wpt_model/attention.py:157-188: q = q_norm(q(x)) per
head, entries = [k_norm(k(x)), v(x)] appended to the cache, exact attention
over every row so far, the output projection) with pre-norm residual blocks,
a SwiGLU feed-forward block and a final norm before the head, as the model's
extend reads it (model.py:456-473: scores = head(final_norm(hidden)), FP32).
RMSNorm's eps is the reference's (layers.py:9).  extend / undo / new_cache
follow the reference's generation protocol through oracle.cache.

A layer may instead be the reference's window layer (WindowAttention,
attention.py:109-151): q = rotate(q_norm(q(x))), entries
[rotate(k_norm(k(x))), v(x)] at the tokens' positions, the window - 1 entries
carried from before (the cache's tail, cache.py:97-108) joined in front,
window attention with a sink per head, and the output times sigmoid(gate(x))
before the output projection.  Or the reference's sparse layer
(SparseAttention, attention.py:191-216): q = q_norm(q(x)), sparse attention
over the keys and values of the last exact layer's table at the rows that
layer chose for each query plus each query's last window rows, a sink per
head, the same gate.  An exact layer chooses (top_k rows) when a sparse layer
follows it (model.py:134-135); the handoff is the last exact layer's
(model.py:411-423).

autocast=True restates the reference's GPU pass instead, which runs under
torch.autocast(bfloat16) (model.py:466): every matrix product takes bf16
inputs, accumulates in FP32 and rounds its output to bf16; RMSNorm of a bf16
input returns bf16 (nn.RMSNorm with an FP32 weight is not cast by autocast:
checked against torch on an MI355X); the residual stream and every
element-wise product stay bf16 (Residuals keeps its sums in the compute dtype,
residuals.py:106-136); the exact and sparse kernels compute in FP32 and
return q's dtype (pytorch_kernels.py:98-121); a window layer's dense
attention takes bf16 scores and bf16 probabilities (attention.py:79-82 under
autocast); the scores are the head's bf16 output .float().

Weights are a dict of tensors (any dtype; used in FP32, or rounded to bf16
once under autocast):
    embedding (V, D); head (V, D); final_norm (D,)
    layers.{i}.attn_norm (D,)   layers.{i}.qkv (H*c + 2c, D): q rows, k, v
    layers.{i}.q_norm (c,)      layers.{i}.k_norm (c,)
    layers.{i}.out (D, H*c)     layers.{i}.ffn_norm (D,)
    layers.{i}.gate_up (2F, D): gate rows, then up rows
    layers.{i}.down (D, F)
    window layers also: layers.{i}.gate (H*c, D), layers.{i}.sink (H,)
    sparse layers: layers.{i}.q (H*c, D) in place of qkv, no k_norm; gate, sink
"""

import torch
import torch.nn.functional as F

from . import attention, cache

EPS = 1e-6


def rms_norm(x, weight):
    return F.rms_norm(x.float(), (x.shape[-1],), weight.float(), EPS)


def bf16_linear(x, weight):
    """An autocast bf16 matrix product: bf16 inputs (weight already holds
    bf16 values), FP32 products and sums, the output rounded to bf16."""
    return (x.to(torch.bfloat16).float() @ weight.T).to(torch.bfloat16)


def bf16_dense_attention(q, k, v, sink, visible, scale):
    """attention.py:74-82 under autocast: the bf16 product q.k rounded to bf16
    before .float(), the probabilities rounded to v's dtype (bf16) before the
    bf16 product with v."""
    z = torch.einsum("...qhc,...kc->...hqk", q.float(), k.float()).to(torch.bfloat16).float() * scale
    z = z.masked_fill(~visible[..., None, :, :], float("-inf"))
    lse = torch.logaddexp(torch.logsumexp(z, -1), sink.float()[:, None])
    p = (z - lse[..., None]).exp().to(torch.bfloat16)
    return torch.einsum("...hqk,...kc->...qhc", p.float(), v.float()).to(torch.bfloat16)


class Decoder:
    def __init__(self, weights, layers, heads, head_dim, kinds=(), window=128, rope_dims=64, rope_base=10000.0,
                 top_k=1024, autocast=False):
        self.autocast = autocast
        if autocast:  # matrices rounded to bf16 once (held as FP32 values); norm weights and sinks FP32
            self.w = {name: value.float() if name.endswith("norm") or name.endswith("sink")
                      else value.to(torch.bfloat16).float() for name, value in weights.items()}
        else:
            self.w = {name: value.float() for name, value in weights.items()}
        self.layers, self.heads, self.head_dim = layers, heads, head_dim
        self.kinds = tuple(kinds) or ("exact",) * layers
        self.window, self.rope_dims, self.rope_base = window, rope_dims, rope_base
        self.top_k = top_k
        # bf16 scores of two implementations may order near ties of the
        # choice another way: a test may give a choosing layer's rows
        # (given[i], (B, T, K) with -1 past a query's rows) for the sparse
        # layers to read instead of the layer's own, after checking them
        # against the layer's own choice kept in choices[i] = (chosen, q,
        # keys, positions) of the last reading
        self.given, self.choices = {}, {}

    def new_cache(self, rows):
        return cache.Rows(rows)

    def _linear(self, x, weight):
        return bf16_linear(x, weight) if self.autocast else x.float() @ weight.T

    def _norm(self, x, weight):
        if self.autocast:  # torch's RMSNorm on the bf16 input, as the reference's module runs it
            return F.rms_norm(x.to(torch.bfloat16), (x.shape[-1],), weight.float(), EPS)
        return rms_norm(x, weight)

    def _layer(self, i, h, reading, handoff):
        """(h after layer i, the handoff for the layers after it)."""
        w = lambda name: self.w[f"layers.{i}.{name}"]  # noqa: E731
        B, T, _ = h.shape
        H, c = self.heads, self.head_dim
        x = self._norm(h, w("attn_norm"))
        positions = reading.positions(T)
        if self.kinds[i] == "sparse":
            q = self._norm(self._linear(x, w("q")).reshape(B, T, H, c), w("q_norm"))
            keys, values, chosen = handoff
            o = attention.sparse_attention(q, keys, values, w("sink"), chosen, positions, c ** -0.5, self.window)
            o = o * torch.sigmoid(self._linear(x, w("gate"))).reshape(B, T, H, c)
            return self._rest(i, h, o), handoff
        qkv = self._linear(x, w("qkv"))
        q = self._norm(qkv[..., :H * c].reshape(B, T, H, c), w("q_norm"))
        k = self._norm(qkv[..., H * c:H * c + c], w("k_norm"))
        v = qkv[..., H * c + c:]
        if self.kinds[i] == "window":
            W = self.window
            q = attention.rotate(q, positions, self.rope_dims, self.rope_base)
            entries = torch.cat([attention.rotate(k, positions, self.rope_dims, self.rope_base), v], -1)
            table = torch.cat([reading.before(("window", i), W - 1, entries), entries], 1)
            if self.autocast:
                visible = attention.window_visible(positions.expand(B, T), W, T)
                o = bf16_dense_attention(q, table[..., :c], table[..., c:], w("sink"), visible, c ** -0.5)
            else:
                o = attention.window_attention(q, table[..., :c], table[..., c:], w("sink"), positions, c ** -0.5, W)
            o = o * torch.sigmoid(self._linear(x, w("gate"))).reshape(B, T, H, c)
        else:
            table = reading.everything(("entries", i), torch.cat([k, v], -1))
            chooses = i + 1 < self.layers and self.kinds[i + 1] == "sparse"
            o, chosen = attention.exact_attention(q, table[..., :c], table[..., c:], positions, c ** -0.5,
                                                  self.top_k if chooses else 0, self.window)
            if chooses:
                self.choices[i] = (chosen, q, table[..., :c], positions)
                chosen = self.given.get(i, chosen)
            handoff = (table[..., :c], table[..., c:], chosen)
        return self._rest(i, h, o), handoff

    def _rest(self, i, h, o):
        """The output projection's residual add, then the feed-forward block."""
        w = lambda name: self.w[f"layers.{i}.{name}"]  # noqa: E731
        B, T, H, c = o.shape
        h = h + self._linear(o.reshape(B, T, H * c), w("out"))
        x = self._norm(h, w("ffn_norm"))
        gate, up = self._linear(x, w("gate_up")).chunk(2, -1)
        return h + self._linear(F.silu(gate) * up, w("down"))

    def extend(self, ids, rows, counts=None, undoable=False, features=()):
        """(scores (B, n, V) FP32, hidden (B, n, D)) of ids (B, n), row b's
        first counts[b] tokens after its earlier ones, the rest padding; with
        features (layer numbers 0 .. layers), also the residual stream
        entering each named layer (`layers`: the final hidden states), FP32,
        side by side in the order named (model.py:406-436, 457-473)."""
        ids = torch.as_tensor(ids, dtype=torch.long)
        counts = torch.full((ids.shape[0],), ids.shape[1]) if counts is None else torch.as_tensor(counts)
        reading = rows.reading(counts, undoable)
        h = self.w["embedding"][ids]
        if self.autocast:
            h = h.to(torch.bfloat16)
        found = {}
        handoff = None
        for i in range(self.layers):
            if i in features:
                found[i] = h.float()
            h, handoff = self._layer(i, h, reading, handoff)
        if self.layers in features:
            found[self.layers] = h.float()
        scores = self._linear(self._norm(h, self.w["final_norm"]), self.w["head"]).float()
        reading.finish()
        if features:
            return scores, h, torch.cat([found[n] for n in features], -1)
        return scores, h

    def forced(self, inputs, rows, counts=None, undoable=True):
        """Each layer run on another pass's residual streams: inputs[i] (B, n,
        D) is the stream entering layer i of that pass (its features), for
        i = 0 .. layers.  Returns (outputs, scores): outputs[i] = layer i's
        output on inputs[i], which that pass gave as inputs[i + 1], and the
        head's scores on inputs[layers].  The new tokens' entries come from
        inputs[i], as that pass wrote them."""
        B, n, _ = inputs[0].shape
        counts = torch.full((B,), n) if counts is None else torch.as_tensor(counts)
        reading = rows.reading(counts, undoable)
        dtype = torch.bfloat16 if self.autocast else torch.float32
        outputs, handoff = [], None
        for i in range(self.layers):
            h, handoff = self._layer(i, inputs[i].to(dtype), reading, handoff)
            outputs.append(h)
        scores = self._linear(self._norm(inputs[self.layers].to(dtype), self.w["final_norm"]), self.w["head"]).float()
        reading.finish()
        return outputs, scores

    def undo(self, rows, kept):
        rows.undo(kept)

    def forward(self, ids):
        """The scores of each row's whole text (B, T, V), read in one pass."""
        ids = torch.as_tensor(ids, dtype=torch.long)
        return self.extend(ids, self.new_cache(ids.shape[0]))[0]
