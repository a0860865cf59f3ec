"""Oracle drafter: the DSpark-shaped drafter restated on the CPU in FP32 (test
infrastructure; see oracle/__init__.py), following the reference's
Drafter.backbone and Drafter.draft (packages/wpt-model/src/wpt_model/
drafter.py:155-234) with the two stand-ins the build's drafter takes: a
dense SwiGLU feed-forward block in place of the routed experts, and plain
pre-norm residual sums in place of Attention Residuals.

    visible     the mask of drafter.py:173-176: place k sees the whole block
                and context entry j where its position lengths - WINDOW + j
                is >= 0 and > the place's position - WINDOW
    backbone    fused = RMSNorm(fuse(context)); x = [embedding(anchor);
                mask ...]; per layer: the window layer's attention over the
                table [block entries ; context entries] (each through the
                layer's own q/k/v projections, norms and rotary encoding, the
                context at positions clamped to >= 0: drafter.py:141-151) with
                the layer's sink, gated, projected, added; then the
                feed-forward block; final norm; U = the target's head
    draft       per place: q = probabilities(U_k + markov_out(markov_in[x_{k-1}])),
                x_k ~ q (the writer's generator), confidence
                sigmoid((w . [h_k ; markov_in[x_{k-1}]] + b) / T_k)
"""

import torch
import torch.nn.functional as F

from . import attention

WINDOW = 128
EPS = 1e-6


def rms_norm(x, weight):
    return F.rms_norm(x.float(), (x.shape[-1],), weight.float(), EPS)


def visible(lengths, count, window=WINDOW):
    """(R, count, count + window) bool over the table [block ; context]."""
    positions = lengths[:, None] + torch.arange(count)
    context_positions = lengths[:, None] - window + torch.arange(window)
    seen = (context_positions[:, None, :] >= 0) & (context_positions[:, None, :] > positions[..., None] - window)
    return torch.cat([torch.ones(len(lengths), count, count, dtype=torch.bool), seen], -1)


class Drafter:
    """weights: wpt_amd.drafter.random_drafter_weights' names (any dtype, used
    in FP32); embedding and head: the target's (V, D)."""

    def __init__(self, weights, embedding, head, layers, heads, head_dim, rope_dims=64, rope_base=10000.0):
        self.w = {name: value.float() for name, value in weights.items()}
        self.embedding, self.head = embedding.float(), head.float()
        self.layers, self.heads, self.head_dim = layers, heads, head_dim
        self.rope_dims, self.rope_base = rope_dims, rope_base

    def _rotate(self, x, positions):
        return attention.rotate(x, positions, self.rope_dims, self.rope_base)

    def _layer(self, i, h, fused, positions, context_positions, mask):
        w = lambda name: self.w[f"layers.{i}.{name}"]  # noqa: E731
        H, c = self.heads, self.head_dim
        x = rms_norm(h, w("attn_norm"))
        proj = x @ w("qkvg").T
        q = self._rotate(rms_norm(proj[..., :H * c].unflatten(-1, (H, c)), w("q_norm")), positions)
        block = torch.cat([self._rotate(rms_norm(proj[..., H * c:H * c + c], w("k_norm")), positions),
                           proj[..., H * c + c:H * c + 2 * c]], -1)
        ctx = fused @ w("qkvg")[H * c:H * c + 2 * c].T
        injected = torch.cat([self._rotate(rms_norm(ctx[..., :c], w("k_norm")), context_positions), ctx[..., c:]], -1)
        table = torch.cat([block, injected], 1)
        o = attention.dense_attention(q, table[..., :c], table[..., c:], w("sink"), mask, c ** -0.5)
        o = o * torch.sigmoid(proj[..., H * c + 2 * c:]).unflatten(-1, (H, c))
        h = h + o.flatten(-2) @ w("out").T
        x = rms_norm(h, w("ffn_norm"))
        gate, up = (x @ w("gate_up").T).chunk(2, -1)
        return h + (F.silu(gate) * up) @ w("down").T

    def backbone(self, context, lengths, anchors, count):
        """(h (R, count, D), U (R, count, V)) in FP32."""
        lengths = torch.as_tensor(lengths, dtype=torch.long)
        R = len(anchors)
        positions = lengths[:, None] + torch.arange(count)
        context_positions = (lengths[:, None] - WINDOW + torch.arange(WINDOW)).clamp(min=0)
        mask = visible(lengths, count)
        fused = rms_norm(context.float() @ self.w["fuse"].T, self.w["fuse_norm"])
        h = torch.cat([self.embedding[anchors][:, None], self.w["mask"].expand(R, count - 1, -1)], 1)
        for i in range(self.layers):
            h = self._layer(i, h, fused, positions, context_positions, mask)
        h = rms_norm(h, self.w["final_norm"])
        return h, h @ self.head.T

    def markov(self, previous):
        embedded = self.w["markov_in"][previous]
        return embedded @ self.w["markov_out"].T, embedded

    def confidence(self, h, embedded, k):
        logit = torch.cat([h, embedded], -1) @ self.w["confidence"].T + self.w["confidence_bias"]
        return torch.sigmoid(logit[..., 0] / self.w["temperatures"][k])

    def distributions(self, context, lengths, anchors, drawn, probabilities):
        """(q (R, count, V), confidences (R, count)) along given drawn tokens
        (R, count): place k's Markov bias reads drawn[:, k - 1] (the anchor at k = 0)."""
        count = drawn.shape[1]
        h, U = self.backbone(context, lengths, anchors, count)
        previous = torch.cat([torch.as_tensor(anchors)[:, None], drawn[:, :-1]], 1)
        qs, confidences = [], []
        for k in range(count):
            bias, embedded = self.markov(previous[:, k])
            qs.append(probabilities(U[:, k] + bias))
            confidences.append(self.confidence(h[:, k], embedded, k))
        return torch.stack(qs, 1), torch.stack(confidences, 1)
