"""An independent numpy forward of the Gemma 4 text decoder (test infrastructure only).

Written from the reference's Rust source, not from oracle/gemma4.c:
crates/gemma4/src/cpu/decoder.rs:334-626 (run_body, layer_forward, attention_forward,
feedforward_forward, project_logits), cpu/attention.rs:206-276, cpu/rotary.rs:33-134,
cpu/norm.rs, cpu/elementwise.rs, config.rs:217-247. It works on the checkpoint-named
BF16 parameters (tests/gemma_oracle.synth_named) and a whole token sequence at once,
vectorized over positions, heads and outputs.

Two arithmetic modes:
- "bf16": FP32 operations with a BF16 rounding at every point where the reference
  rounds (the eager policy); FP32 sums run sequentially (np.cumsum) as the Rust loops do.
- "fp64": the same equations in float64 with no rounding at all (the parameters are
  the BF16 values). It differs from the eager decoder only by BF16 rounding noise.
"""
import numpy as np

PREFIX = "model.language_model."


def _bf16(x):
    """float32 -> nearest-even bfloat16 value (as float32); NaN -> canonical NaN."""
    x = np.asarray(x, np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32)
    r = np.where(np.isnan(x), np.uint32(0x7FC0), r)
    return (r << 16).astype(np.uint32).view(np.float32)


def _as_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


class Arith:
    def __init__(self, mode):
        assert mode in ("bf16", "fp64")
        self.mode = mode
        self.dt = np.float32 if mode == "bf16" else np.float64

    def r(self, x):
        """A reference rounding point."""
        return _bf16(x) if self.mode == "bf16" else np.asarray(x, np.float64)

    def f(self, x):
        return np.asarray(x, self.dt)

    def seqsum(self, x, axis=-1):
        """Sequential left-to-right sum (Rust loops) in bf16 mode; exact-order irrelevant in fp64."""
        if self.mode == "bf16":
            return np.take(np.cumsum(np.asarray(x, np.float32), axis=axis, dtype=np.float32), -1, axis=axis)
        return np.sum(x, axis=axis)


def _params(named, dt):
    return {k[len(PREFIX):] if k.startswith(PREFIX) else k: _as_f32(v).astype(dt) for k, v in named.items()}


class GemmaNumpy:
    """Gemma 4 text decoder over a whole sequence (prefill semantics: logits of every position).

    cfg fields: vocab, hidden, heads, kv_heads, ple, eps, softcap, window, kinds ("S"/"F" per layer),
    head_dim (per layer), theta (per layer), proportional (per layer), kv_owner (per layer)."""

    def __init__(self, cfg, named, mode="bf16"):
        self.c = cfg
        self.a = Arith(mode)
        self.p = _params(named, self.a.dt)

    # -- operations, each named after the reference function it follows
    def project(self, x, w):
        """cpu/linear.rs:23-66: out[r][c] = round(sum_k x[r][k] w[c][k]) (FP32, k ascending)."""
        a = self.a
        if a.mode == "bf16":
            prod = (x[:, None, :].astype(np.float32) * w[None, :, :].astype(np.float32))
            return a.r(a.seqsum(prod, axis=-1))
        return x @ w.T

    def rms(self, x, width, scale=None):
        """cpu/norm.rs normalize: FP32 energy, (mean + eps)^-1/2, x * inverse (* scale), one rounding."""
        a = self.a
        rows = x.reshape(-1, width)
        energy = a.seqsum(rows * rows, axis=-1)
        mean = energy / a.f(width)
        inverse = a.f(np.power(mean + a.f(self.c.eps), a.f(-0.5)))
        v = rows * inverse[:, None]
        if scale is not None:
            v = v * scale[None, :]
        return a.r(v).reshape(x.shape)

    def scale(self, x, factor):
        return self.a.r(x * self.a.f(factor))

    def gelu(self, x):
        """elementwise.rs gelu_tanh: 0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2)))."""
        a = self.a
        alpha, cubic = a.f(0.7978846), a.f(0.044715)
        inner = alpha * x * (a.f(1) + cubic * x * x)
        return a.r(a.f(0.5) * x * (a.f(1) + np.tanh(inner)))

    def softcap(self, x):
        a = self.a
        cap = a.f(self.c.softcap)
        return a.r(a.r(np.tanh(a.r(x / cap))) * cap)

    def inv_freq(self, layer):
        """config.rs:217-247: 1 / theta^(2p / width) in FP32; proportional layers keep pairs/4."""
        a = self.a
        width = self.c.head_dim[layer]
        pairs = width // 2
        active = pairs // 4 if self.c.proportional[layer] else pairs
        p = np.arange(pairs)
        exponent = a.f(p * 2) / a.f(width)
        inv = a.f(1) / np.power(a.f(self.c.theta[layer]), exponent)
        return np.where(p < active, inv, a.f(0))

    def rotary(self, x, heads, width, positions, layer):
        """rotary.rs factors + apply_rotary: BF16 cos/sin of position * frequency; each product rounded,
        the sum rounded. x: [seq, heads * width]."""
        a = self.a
        half = width // 2
        phase = a.f(positions)[:, None] * self.inv_freq(layer)[None, :]
        cos, sin = a.r(np.cos(phase)), a.r(np.sin(phase))
        x = x.reshape(len(positions), heads, width)
        lo, hi = x[..., :half], x[..., half:]
        c, s = cos[:, None, :], sin[:, None, :]
        first = a.r(lo * c) + a.r(-hi * s)
        second = a.r(hi * c) + a.r(lo * s)
        return np.concatenate([a.r(first), a.r(second)], axis=-1).reshape(len(positions), heads * width)

    def attention(self, q, keys, values, width, window, positions):
        """cpu/attention.rs: BF16 scores, FP32 softmax, BF16 weights, FP32 weight x value accumulation."""
        a, c = self.a, self.c
        groups = c.heads // c.kv_heads
        seq = q.shape[0]
        q = q.reshape(seq, c.heads, width)
        k = keys.reshape(-1, c.kv_heads, width)
        v = values.reshape(-1, c.kv_heads, width)
        out = np.zeros((seq, c.heads, width), a.dt)
        for i, pos in enumerate(positions):
            first = 0 if window is None else max(0, pos - (window - 1))
            kk, vv = k[first:pos + 1], v[first:pos + 1]
            for h in range(c.heads):
                kh = h // groups
                scores = a.r(a.seqsum(q[i, h][None, :] * kk[:, kh, :], axis=-1))
                e = np.exp(scores - scores.max())
                total = a.seqsum(e)
                w = a.r(e / total)
                out[i, h] = a.r(a.seqsum(w[:, None] * vv[:, kh, :], axis=0))
        return out.reshape(seq, c.heads * width)

    # -- the decoder (decoder.rs:334-626)
    def forward(self, tokens):
        """Post-soft-cap logits of every position of `tokens` (a fresh sequence)."""
        a, c, P = self.a, self.c, self.p
        seq, H, ple, L = len(tokens), c.hidden, c.ple, len(c.kinds)
        tokens = np.asarray(tokens)
        positions = np.arange(seq)
        embed_scale = a.r(a.f(np.sqrt(np.float32(H)))) if a.mode == "bf16" else np.sqrt(H)
        ple_scale = a.r(a.f(np.sqrt(np.float32(ple)))) if a.mode == "bf16" else np.sqrt(ple)
        proj_scale = a.f(1) / a.f(np.sqrt(a.f(H)))
        hidden = self.scale(P["embed_tokens.weight"][tokens], embed_scale)
        identity = self.scale(P["embed_tokens_per_layer.weight"][tokens], ple_scale)
        projection = self.scale(self.project(hidden, P["per_layer_model_projection.weight"]), proj_scale)
        per_layer = []
        for l in range(L):
            sl = projection[:, l * ple:(l + 1) * ple]
            context = self.rms(sl, ple, P["per_layer_projection_norm.weight"])
            combined = a.r(context + identity[:, l * ple:(l + 1) * ple])
            per_layer.append(self.scale(combined, 0.70710677))
        caches = {}
        for l in range(L):
            hidden = self.layer(l, hidden, per_layer[l], positions, caches)
        last = self.rms(hidden[-1:], H, P["norm.weight"])
        return self.softcap(self.project(last, P["embed_tokens.weight"]))[0], hidden

    def layer(self, l, hidden, per_layer, positions, caches):
        a, c, P = self.a, self.c, self.p
        pre = f"layers.{l}."
        H, width = c.hidden, c.head_dim[l]
        normed = self.rms(hidden, H, P[pre + "input_layernorm.weight"])
        q = self.project(normed, P[pre + "self_attn.q_proj.weight"])
        q = self.rms(q, width, P[pre + "self_attn.q_norm.weight"])
        q = self.rotary(q, c.heads, width, positions, l)
        if c.kv_owner[l] == l:
            k = self.project(normed, P[pre + "self_attn.k_proj.weight"])
            k = self.rms(k, width, P[pre + "self_attn.k_norm.weight"])
            k = self.rotary(k, c.kv_heads, width, positions, l)
            v = self.project(normed, P[pre + "self_attn.v_proj.weight"])
            v = self.rms(v, width)
            caches[l] = (k, v)
        keys, values = caches[c.kv_owner[l]]
        window = c.window if c.kinds[l] == "S" else None
        attended = self.attention(q, keys, values, width, window, positions)
        projected = self.project(attended, P[pre + "self_attn.o_proj.weight"])
        hidden = a.r(hidden + self.rms(projected, H, P[pre + "post_attention_layernorm.weight"]))
        # feed-forward
        residual = hidden
        normed = self.rms(hidden, H, P[pre + "pre_feedforward_layernorm.weight"])
        gate = self.project(normed, P[pre + "mlp.gate_proj.weight"])
        up = self.project(normed, P[pre + "mlp.up_proj.weight"])
        product = a.r(self.gelu(gate) * up)
        down = self.project(product, P[pre + "mlp.down_proj.weight"])
        hidden = a.r(residual + self.rms(down, H, P[pre + "post_feedforward_layernorm.weight"]))
        # per-layer input
        residual = hidden
        gate = self.project(hidden, P[pre + "per_layer_input_gate.weight"])
        product = a.r(self.gelu(gate) * per_layer)
        projected = self.project(product, P[pre + "per_layer_projection.weight"])
        hidden = a.r(residual + self.rms(projected, H, P[pre + "post_per_layer_input_norm.weight"]))
        return self.scale(hidden, P[pre + "layer_scalar"][0])


class Cfg:
    """The numpy forward's view of a gemma_oracle.config()."""

    def __init__(self, c):
        n = c.layers
        self.vocab, self.hidden, self.heads, self.kv_heads, self.ple = c.vocab, c.hidden, c.heads, c.kv_heads, c.ple
        self.eps, self.softcap, self.window = c.eps, c.softcap, c.window
        self.kinds = ["F" if c.kind[i] else "S" for i in range(n)]
        self.head_dim = [c.head_dim[i] for i in range(n)]
        self.theta = [c.theta[i] for i in range(n)]
        self.proportional = [bool(c.proportional[i]) for i in range(n)]
        self.kv_owner = [c.kv_owner[i] for i in range(n)]
