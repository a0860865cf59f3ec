"""A DSpark-shaped drafter for the speculative writer, on the GPU: the
reference's Drafter.draft (packages/wpt-model/src/wpt_model/drafter.py:
155-234) over this build's decoder.

One round drafts `count` tokens after each row's anchor (the last token
written, not yet read):

    context   the residual streams of the target's feature layers at each of
              the last WINDOW tokens the model read (the Writer keeps them:
              wpt_amd.writer), fused: RMSNorm(fuse(context))
    backbone  `layers` layers, each a window layer's attention over the block
              and the fused context (the context enters every layer as keys
              and values through that layer's own key/value projection, with
              rotary encoding at the context tokens' positions), then a
              feed-forward block; the block is the anchor's embedding then a
              mask vector per later place; each place sees the whole block
              and the context entries at positions >= 0 within WINDOW tokens
              before it (drafter.py:173-176)
    head      the target's own output head on the final norm: base scores U_k
    Markov    q_k = probabilities(U_k + markov_out(markov_in[x_{k-1}])), the
              writer's distribution (temperature, top-k); x_0 the anchor;
              x_k drawn from q_k with the writer's generator (drafter.py:215-234)
    confidence c_k = sigmoid((w . [h_k ; markov_in[x_{k-1}]] + b) / T_k)

What differs from the reference, by design: the feed-forward block is a dense
SwiGLU block in place of the routed experts, and the sublayers are linked by
plain pre-norm residual sums in place of Attention Residuals (the same two
stand-ins as wpt_amd.decoder's layout of a WPT model).  Like the reference,
the backbone runs in bf16 and the Markov and confidence heads in FP32.

On the GPU: the projections and the head on wptv_gemm (the build's MFMA
product) up to 512 rows, the context fuse (R x WINDOW rows) on torch's; the
attention on wptv_verify_attention's row-block kernel, with the table laid
out as [context ; block] and each place's position chosen so that the
kernel's window is exactly what the reference's mask shows it; norms, rotary
encoding and sampling in torch (small tensors).  With capture=True the
backbone of each (rows, count) shape is captured once in a HIP graph and
replayed on copies of its inputs (the same kernels, so the same results).
"""

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import kernels, layers

WINDOW = 128        # the context's tokens (attention.py:53; drafter.window)
BLOCK = 5           # the most drafts per round (drafter.py:72)
LAYERS = 3          # the production backbone's layers (drafter.py:73)
MARKOV_RANK = 256   # the Markov head's rank at a width of 4096 (drafter.py:74-75)
MARKOV_WIDTH = 4096
FEATURES = 5        # target layers read (drafter.py:76)
EPS = 1e-6


def feature_layers(n_layer, count=FEATURES):
    """The target layers (numbered from 1) a drafter reads: `count` of them
    spread evenly from the 2nd to the third-to-last, fewer where the model
    has fewer there (drafter.py:80-87)."""
    first, last = 2, min(max(2, n_layer - 2), n_layer)
    if count == 1 or first == last:
        return (first,)
    return tuple(sorted({round(first + i * (last - first) / (count - 1)) for i in range(count)}))


def default_markov_rank(width):
    return max(1, MARKOV_RANK * width // MARKOV_WIDTH)


@dataclass(frozen=True)
class DrafterConfig:
    features: tuple
    layers: int = LAYERS
    block: int = BLOCK
    markov_rank: int = MARKOV_RANK
    ffn: int = 0  # the dense feed-forward block's width (0: the target's)

    @classmethod
    def for_model(cls, model_config, features=None, layers=LAYERS, block=BLOCK, markov_rank=None, ffn=0):
        features = tuple(features) if features is not None else feature_layers(model_config.layers)
        if any(not 1 <= n <= model_config.layers for n in features):
            raise ValueError(f"drafter config: features {list(features)} are not layers 1 .. {model_config.layers}")
        return cls(features, layers, block, markov_rank or default_markov_rank(model_config.d_model),
                   ffn or model_config.ffn)


def random_drafter_weights(model_config, config, seed=0, std=0.02, device="cpu"):
    """Random-init drafter weights in FP32, drawn in a fixed order from one
    seeded generator: every matrix ~ N(0, std), the mask vector ~ N(0, 1)
    (the embedding's scale), norms 1, sinks ~ N(0, 1), the Markov output
    zero (the reference starts it at zero: drafter.py:170), temperatures 1."""
    generator = torch.Generator(device=device).manual_seed(seed)
    D, H, c, V = model_config.d_model, model_config.heads, model_config.head_dim, model_config.vocab
    F_, r = config.ffn, config.markov_rank

    def normal(*shape, scale=std):
        return torch.randn(*shape, generator=generator, device=device) * scale

    ones = lambda n: torch.ones(n, device=device)  # noqa: E731
    w = {"fuse": normal(D, len(config.features) * D), "fuse_norm": ones(D), "mask": normal(D, scale=1.0)}
    for i in range(config.layers):
        w[f"layers.{i}.attn_norm"] = ones(D)
        w[f"layers.{i}.qkvg"] = normal(2 * H * c + 2 * c, D)  # q, k, v, gate rows
        w[f"layers.{i}.q_norm"], w[f"layers.{i}.k_norm"] = ones(c), ones(c)
        w[f"layers.{i}.sink"] = normal(H, scale=1.0)
        w[f"layers.{i}.out"] = normal(D, H * c)
        w[f"layers.{i}.ffn_norm"] = ones(D)
        w[f"layers.{i}.gate_up"] = normal(2 * F_, D)
        w[f"layers.{i}.down"] = normal(D, F_)
    w["final_norm"] = ones(D)
    w["markov_in"] = normal(V, r, scale=1.0)
    w["markov_out"] = torch.zeros(V, r, device=device)
    w["confidence"] = normal(1, D + r)
    w["confidence_bias"] = torch.zeros(1, device=device)
    w["temperatures"] = torch.ones(config.block, device=device)
    return w


def visible_positions(lengths, count, window=WINDOW):
    """The positions each place's query takes so that the row-block kernel
    (rows max(0, p - span + 1) .. min(p, N - 1), N = window + count, span =
    N - 1) reads exactly what the reference's mask shows it over the table
    [context ; block]: the whole block, and the context rows j > k (within
    `window` tokens before place k) whose positions lengths - window + j are
    >= 0.  Returns (positions (R, count) int64, span)."""
    N = window + count
    k = torch.arange(count, device=lengths.device)
    first = torch.maximum(k[None] + 1, (window - lengths)[:, None])  # the first context row place k reads
    return first + N - 2, N - 1


class Drafter:
    """features, window: what the Writer reads (the drafter protocol,
    wpt_inference/__init__.py:17-33); draft() proposes tokens."""

    def __init__(self, model, config, weights, capture=False):
        self.model, self.config = model, config
        self.capture = capture
        self._graphs = {}  # (rows, count) -> (graph, its inputs, its outputs)
        self.features, self.window, self.block = config.features, WINDOW, config.block
        mc = model.config
        self.heads, self.head_dim = mc.heads, mc.head_dim
        dev = model.device
        fp32 = ("norm", "sink", "markov_in", "markov_out", "confidence", "confidence_bias", "temperatures")
        self.w = {name: value.to(device=dev, dtype=torch.float32 if name.endswith(fp32) else torch.bfloat16)
                  .contiguous() for name, value in weights.items()}
        self.divisors = layers.rope_divisors(mc.rope_dims, mc.rope_base, dev)
        self.rope_dims = mc.rope_dims

    def _rotate(self, x, positions):
        """Rotary encoding of the last rope_dims of x (R, T, [H,] d) at
        positions (R, T), FP32 angles from the reference's divisors, in x's dtype."""
        angles = positions.float()[..., None] / self.divisors
        cos, sin = angles.cos(), angles.sin()
        if x.dim() == 4:
            cos, sin = cos[..., None, :], sin[..., None, :]
        kept, turning = x[..., :-self.rope_dims], x[..., -self.rope_dims:].float()
        even, odd = turning[..., 0::2], turning[..., 1::2]
        turned = torch.stack([even * cos - odd * sin, even * sin + odd * cos], -1).flatten(-2)
        return torch.cat([kept, turned.to(x.dtype)], -1)

    @staticmethod
    def _linear(x, w):
        if x.numel() // x.shape[-1] <= layers.LINEAR_MAX_ROWS:
            return layers.linear(x, w)
        return F.linear(x, w)

    @staticmethod
    def _norm(x, weight):
        """RMSNorm of x's rows times weight (FP32 math, one rounding to x's
        dtype, as torch's rms_norm of a bf16 x and an FP32 weight): the
        library's one-launch kernel for contiguous bf16 rows, torch otherwise."""
        if x.dtype == torch.bfloat16 and x.is_contiguous() and x.shape[-1] % 8 == 0 and x.shape[-1] <= 4096:
            return layers.add_rms_norm(x, None, weight, torch.empty_like(x), EPS)
        return F.rms_norm(x, (x.shape[-1],), weight, EPS)

    def _heads_norm(self, x, weight, heads, positions):
        """RMSNorm of each of the first heads * c columns' heads of x (R, T,
        width), times weight (c,), then the rotary encoding at positions (R,
        T): (R, T, heads, c), one launch."""
        if x.dtype == torch.bfloat16 and weight.shape[0] in (64, 128, 256):
            return layers.heads_rms_norm(x, weight, heads, EPS, positions=positions, divisors=self.divisors)
        normed = self._norm(x[..., :heads * weight.shape[0]].unflatten(-1, (heads, weight.shape[0])), weight)
        return self._rotate(normed, positions)

    def _layer(self, i, h, fused, positions, context_positions, places, span):
        w = lambda name: self.w[f"layers.{i}.{name}"]  # noqa: E731
        R, count, D = h.shape
        H, c = self.heads, self.head_dim
        x = self._norm(h, w("attn_norm"))
        proj = self._linear(x, w("qkvg"))  # (R, count, (2H + 2) c): q, k, v, gate
        q = self._heads_norm(proj, w("q_norm"), H, positions)
        block = torch.cat([self._heads_norm(proj[..., H * c:], w("k_norm"), 1, positions)[..., 0, :],
                           proj[..., H * c + c:H * c + 2 * c]], -1)
        kv = w("qkvg")[H * c:H * c + 2 * c]  # the layer's own key/value projection injects the context
        ctx = self._linear(fused, kv)  # (R, WINDOW, 2c)
        injected = torch.cat([self._heads_norm(ctx, w("k_norm"), 1, context_positions)[..., 0, :], ctx[..., c:]], -1)
        table = torch.cat([injected, block], 1).contiguous()  # [context ; block]
        o = kernels.verify_attention(q.contiguous(), table[..., :c], table[..., c:], places, c ** -0.5, window=span,
                                     sink=w("sink"))
        gated = o * torch.sigmoid(proj[..., H * c + 2 * c:]).unflatten(-1, (H, c))
        h = h + self._linear(gated.flatten(-2), w("out"))
        x = self._norm(h, w("ffn_norm"))
        gate, up = self._linear(x, w("gate_up")).chunk(2, -1)
        return h + self._linear(F.silu(gate) * up, w("down"))

    @torch.no_grad()
    def backbone(self, context, lengths, anchors, count):
        """(h (R, count, D) FP32, U (R, count, V) FP32): context (R, WINDOW,
        features * D) FP32, lengths (R,) the anchors' positions, anchors (R,)."""
        if not 1 <= count <= self.block:
            raise ValueError(f"the drafter drafts 1 to {self.block} tokens, not {count}")
        R = anchors.shape[0]
        dev = anchors.device
        lengths = lengths.to(device=dev, dtype=torch.long)
        positions = lengths[:, None] + torch.arange(count, device=dev)
        context_positions = (lengths[:, None] - WINDOW + torch.arange(WINDOW, device=dev)).clamp(min=0)
        places, span = visible_positions(lengths, count)
        fused = self._norm(self._linear(context.to(torch.bfloat16), self.w["fuse"]), self.w["fuse_norm"])
        embedding = self.model.w["embedding"]
        x = torch.cat([embedding[anchors][:, None].to(torch.bfloat16),
                       self.w["mask"].expand(R, count - 1, -1)], 1)
        h = x
        for i in range(self.config.layers):
            h = self._layer(i, h, fused, positions, context_positions, places, span)
        h = self._norm(h, self.w["final_norm"])
        return h.float(), self._linear(h, self.model.w["head"]).float()

    def _replayed(self, features, lengths, anchors, count):
        """backbone() from its HIP graph for this shape; the first call of a
        shape runs eagerly (which also readies the libraries it calls) and then
        captures the graph (which runs nothing).  A replay's outputs are the
        graph's own tensors, valid until the next replay."""
        key = (anchors.shape[0], count)
        if key not in self._graphs:
            eager = self.backbone(features, lengths, anchors, count)
            inputs = (torch.zeros_like(features, dtype=torch.float32), torch.zeros_like(lengths, dtype=torch.long),
                      torch.zeros_like(anchors))
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                outputs = self.backbone(*inputs, count)
            self._graphs[key] = (graph, inputs, outputs)
            return eager
        graph, (f_in, l_in, a_in), outputs = self._graphs[key]
        f_in.copy_(features)
        l_in.copy_(lengths)
        a_in.copy_(anchors)
        graph.replay()
        return outputs

    def _markov(self, previous):
        embedded = self.w["markov_in"][previous]
        return embedded @ self.w["markov_out"].T, embedded

    @torch.no_grad()
    def draft(self, model, histories, context, count, probabilities, generator):
        """The drafter protocol: (tokens (R, count), their distributions
        (R, count, V), confidences (R, count)), each token drawn from its
        distribution with the writer's generator."""
        features, lengths = context
        anchors = torch.tensor([history[-1] for history in histories], dtype=torch.long, device=self.model.device)
        if self.capture:
            h, U = self._replayed(features, lengths, anchors, count)
        else:
            h, U = self.backbone(features, lengths, anchors, count)
        tokens, distributions, confidences = [], [], []
        previous = anchors
        for k in range(count):
            bias, embedded = self._markov(previous)
            q = probabilities(U[:, k] + bias)
            previous = torch.multinomial(q, 1, generator=generator)[:, 0]
            logit = torch.cat([h[:, k], embedded], -1) @ self.w["confidence"].T + self.w["confidence_bias"]
            confidences.append(torch.sigmoid(logit[:, 0] / self.w["temperatures"][k]))
            tokens.append(previous)
            distributions.append(q)
        return torch.stack(tokens, 1), torch.stack(distributions, 1), torch.stack(confidences, 1)
