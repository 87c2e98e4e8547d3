"""ctypes binding of the Gemma 4 CPU decoder restatement (oracle/gemma4.c) -- test and
benchmark infrastructure only -- plus the configs[0] tiny model: its configuration
and seeded synthetic BF16 weights.

The tiny configuration follows BASELINE configs[0]: hidden 512, 4 layers, 8 query
heads, 2 KV heads, head_dim 64, FFN 2048, vocab 32000, eps 1e-6, RoPE theta 1e4.
Gemma 4 fields that BASELINE leaves open are fixed here:
- per-layer input width (PLE) 64, PLE vocabulary 32000;
- no shared-KV layers;
- soft cap 30;
- context 128;
- sliding window 512, so every sliding layer attends to the full causal prefix at these lengths;
- layer types sliding, sliding, sliding, full. The reference's config loader requires the last layer to be full attention (gemma4/src/config.rs:330-335);
- the full layer uses head_dim 64 with quarter-proportional RoPE at theta 1e4.

Weights are N(0, 0.02) from numpy's default_rng(0), drawn tensor by tensor in the
reference's parameter order (parameters.rs:106-160) and rounded to BF16. Norm
weights and layer scalars are 1.0.
"""
import ctypes
import json
import os
import struct

import numpy as np

import oracle_ffi

MAXL = 64


class G4Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("vocab", "hidden", "intermediate", "heads", "kv_heads", "ple", "ple_vocab", "context", "window",
                 "layers")] + [
        ("eps", ctypes.c_float), ("softcap", ctypes.c_float),
        ("kind", ctypes.c_int32 * MAXL), ("head_dim", ctypes.c_int32 * MAXL), ("kv_owner", ctypes.c_int32 * MAXL),
        ("proportional", ctypes.c_int32 * MAXL), ("theta", ctypes.c_float * MAXL)]


LAYER_FIELDS = ("q", "k", "v", "o", "q_norm", "k_norm", "input_norm", "post_attention_norm", "pre_feedforward_norm",
                "post_feedforward_norm", "gate", "up", "down", "ple_gate", "ple_projection", "post_ple_norm",
                "layer_scalar")


class G4LayerWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in LAYER_FIELDS]


class G4Weights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("embed", "ple_embed", "ple_projection", "ple_norm", "final_norm")] + [
        ("layer", G4LayerWeights * MAXL)]


_u16p = ctypes.POINTER(ctypes.c_uint16)


def lib():
    L = oracle_ffi.lib()
    if getattr(L, "_g4_ready", False):
        return L
    c = ctypes
    L.g4_bf16.restype = c.c_uint16
    L.g4_bf16.argtypes = [c.c_float]
    L.g4_project.argtypes = [c.c_void_p, c.c_int, c.c_int, c.c_void_p, c.c_int, c.c_void_p]
    L.g4_set_threads.argtypes = [c.c_int]
    L.g4_rms_norm.argtypes = [c.c_void_p, c.c_int, c.c_int, c.c_float, c.c_void_p, c.c_void_p]
    for f in (L.g4_add, L.g4_multiply):
        f.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p]
    L.g4_scale.argtypes = [c.c_void_p, c.c_size_t, c.c_float, c.c_void_p]
    L.g4_gelu_tanh.argtypes = [c.c_void_p, c.c_size_t, c.c_void_p]
    L.g4_softcap.argtypes = [c.c_void_p, c.c_size_t, c.c_float, c.c_void_p]
    L.g4_ple_combine.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p]
    L.g4_inverse_frequency.argtypes = [c.POINTER(G4Config), c.c_int, c.c_int, c.POINTER(c.c_float)]
    L.g4_factors.argtypes = [c.POINTER(G4Config), c.c_int, c.c_void_p, c.c_int, c.c_void_p, c.c_void_p]
    L.g4_apply_rotary.argtypes = [c.c_void_p, c.c_int, c.c_int, c.c_int, c.c_void_p, c.c_void_p, c.c_void_p]
    L.g4_attention.argtypes = [c.c_void_p, c.c_int, c.c_void_p, c.c_void_p, c.c_int, c.c_int, c.c_int, c.c_int,
                               c.c_int, c.c_int, c.c_int, c.c_void_p, c.c_void_p]
    L.g4_argmax.restype = c.c_int64
    L.g4_argmax.argtypes = [c.c_void_p, c.c_int]
    L.g4_open.restype = c.c_void_p
    L.g4_open.argtypes = [c.POINTER(G4Config), c.POINTER(G4Weights), c.c_char_p, c.c_size_t]
    L.g4_close.argtypes = [c.c_void_p]
    L.g4_reset.argtypes = [c.c_void_p]
    L.g4_position.argtypes = [c.c_void_p]
    L.g4_step.argtypes = [c.c_void_p, c.c_void_p, c.c_int, c.c_void_p]
    L._g4_ready = True
    return L


def set_threads(n):
    """Worker threads of g4_project (default 1, the reference's loops); results do not depend on it."""
    lib().g4_set_threads(int(n))


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def bf16(x):
    """FP32 -> BF16 bits, round to nearest even (NaN -> 0x7fc0), as cpu/linear.rs:10-16."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def load(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def config(vocab=32000, hidden=512, intermediate=2048, heads=8, kv_heads=2, head_dim=64, global_head_dim=64,
           ple=64, ple_vocab=None, context=128, window=512, layers=("S", "S", "S", "F"), shared=0, eps=1e-6,
           softcap=30.0, theta_local=1e4, theta_global=1e4):
    """A normalized Gemma 4 text config (gemma4/src/config.rs:297-380): layer kinds, owners of
    shared tail layers (the last owner of the same kind), per-kind head width and RoPE."""
    c = G4Config()
    c.vocab, c.hidden, c.intermediate, c.heads, c.kv_heads = vocab, hidden, intermediate, heads, kv_heads
    c.ple, c.ple_vocab, c.context, c.window, c.layers = ple, ple_vocab or vocab, context, window, len(layers)
    c.eps, c.softcap = eps, softcap
    owners = len(layers) - shared
    for i, k in enumerate(layers):
        full = k == "F"
        c.kind[i] = 1 if full else 0
        c.head_dim[i] = global_head_dim if full else head_dim
        c.proportional[i] = 1 if full else 0
        c.theta[i] = theta_global if full else theta_local
        c.kv_owner[i] = i if i < owners else max(j for j in range(owners) if layers[j] == k)
    return c


LAYER_SUFFIX = {"q": "self_attn.q_proj.weight", "k": "self_attn.k_proj.weight", "v": "self_attn.v_proj.weight",
                "o": "self_attn.o_proj.weight", "q_norm": "self_attn.q_norm.weight",
                "k_norm": "self_attn.k_norm.weight", "input_norm": "input_layernorm.weight",
                "post_attention_norm": "post_attention_layernorm.weight",
                "pre_feedforward_norm": "pre_feedforward_layernorm.weight",
                "post_feedforward_norm": "post_feedforward_layernorm.weight", "gate": "mlp.gate_proj.weight",
                "up": "mlp.up_proj.weight", "down": "mlp.down_proj.weight",
                "ple_gate": "per_layer_input_gate.weight", "ple_projection": "per_layer_projection.weight",
                "post_ple_norm": "post_per_layer_input_norm.weight", "layer_scalar": "layer_scalar"}
PREFIX = "model.language_model."


def synth_named(c, seed=0, std=0.02):
    """Seeded BF16 parameters for config c, keyed by checkpoint name, in the reference's parameter
    order (parameters.rs:106-160): N(0, std) matrices, 1.0 norms and layer scalars."""
    rng = np.random.default_rng(seed)
    out = {}

    def normal(name, *shape):
        out[PREFIX + name] = bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).reshape(shape)

    def ones(name, n):
        out[PREFIX + name] = np.full(n, 0x3F80, np.uint16)

    H, F, P, L = c.hidden, c.intermediate, c.ple, c.layers
    normal("embed_tokens.weight", c.vocab, H)
    normal("embed_tokens_per_layer.weight", c.ple_vocab, L * P)
    normal("per_layer_model_projection.weight", L * P, H)
    ones("per_layer_projection_norm.weight", P)
    ones("norm.weight", H)
    for l in range(L):
        hd = c.head_dim[l]
        lp = f"layers.{l}."
        shapes = {"q": (c.heads * hd, H), "k": (c.kv_heads * hd, H), "v": (c.kv_heads * hd, H),
                  "o": (H, c.heads * hd), "q_norm": hd, "k_norm": hd, "input_norm": H, "post_attention_norm": H,
                  "pre_feedforward_norm": H, "post_feedforward_norm": H, "gate": (F, H), "up": (F, H),
                  "down": (H, F), "ple_gate": (P, H), "ple_projection": (H, P), "post_ple_norm": H,
                  "layer_scalar": 1}
        for field in LAYER_FIELDS:
            shp = shapes[field]
            if isinstance(shp, tuple):
                normal(lp + LAYER_SUFFIX[field], *shp)
            else:
                ones(lp + LAYER_SUFFIX[field], shp)
    return out


def weights_from_named(c, named):
    """G4Weights pointing into the named arrays (which must stay alive)."""
    w = G4Weights()
    w.embed = ptr(named[PREFIX + "embed_tokens.weight"])
    w.ple_embed = ptr(named[PREFIX + "embed_tokens_per_layer.weight"])
    w.ple_projection = ptr(named[PREFIX + "per_layer_model_projection.weight"])
    w.ple_norm = ptr(named[PREFIX + "per_layer_projection_norm.weight"])
    w.final_norm = ptr(named[PREFIX + "norm.weight"])
    for l in range(c.layers):
        for field in LAYER_FIELDS:
            setattr(w.layer[l], field, ptr(named[PREFIX + f"layers.{l}." + LAYER_SUFFIX[field]]))
    return w


def synth_weights(c, seed=0, std=0.02):
    """Seeded BF16 weights for config c; returns (G4Weights, keepalive)."""
    named = synth_named(c, seed, std)
    return weights_from_named(c, named), named


def config_json(c, layer_kinds, shared=0):
    """The package's config.json for config c (the fields Gemma4Config::from_json reads)."""
    kinds = ["full_attention" if k == "F" else "sliding_attention" for k in layer_kinds]
    local = next((c.head_dim[i] for i in range(c.layers) if not c.kind[i]), c.head_dim[0])
    glob = next((c.head_dim[i] for i in range(c.layers) if c.kind[i]), c.head_dim[0])
    tl = next((float(c.theta[i]) for i in range(c.layers) if not c.kind[i]), 1e4)
    tg = next((float(c.theta[i]) for i in range(c.layers) if c.kind[i]), 1e4)
    text = {"model_type": "gemma4_text", "dtype": "bfloat16", "attention_bias": False, "attention_dropout": 0.0,
            "attention_k_eq_v": False, "bos_token_id": 2, "eos_token_id": 1, "pad_token_id": 0,
            "enable_moe_block": False, "final_logit_softcapping": float(c.softcap), "global_head_dim": glob,
            "head_dim": local, "hidden_activation": "gelu_pytorch_tanh", "hidden_size": c.hidden,
            "hidden_size_per_layer_input": c.ple, "initializer_range": 0.02, "intermediate_size": c.intermediate,
            "layer_types": kinds, "max_position_embeddings": c.context, "num_attention_heads": c.heads,
            "num_hidden_layers": c.layers, "num_key_value_heads": c.kv_heads, "num_kv_shared_layers": shared,
            "rms_norm_eps": float(c.eps), "sliding_window": c.window,
            "rope_parameters": {"sliding_attention": {"rope_type": "default", "rope_theta": tl},
                                "full_attention": {"rope_type": "proportional", "rope_theta": tg,
                                                   "partial_rotary_factor": 0.25}},
            "tie_word_embeddings": True, "use_bidirectional_attention": None, "use_cache": True,
            "use_double_wide_mlp": False, "vocab_size": c.vocab, "vocab_size_per_layer_input": c.ple_vocab,
            "num_global_key_value_heads": None}
    return {"architectures": ["Gemma4ForConditionalGeneration"], "model_type": "gemma4", "dtype": "bfloat16",
            "tie_word_embeddings": True, "image_token_id": c.vocab + 1, "audio_token_id": c.vocab + 2,
            "video_token_id": c.vocab + 3, "text_config": text}


def write_package(directory, c, named, layer_kinds, shared=0):
    """config.json + model.safetensors (BF16 tensors, SafeTensors layout: u64 header length,
    JSON header, 8-byte aligned, then the data)."""
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(config_json(c, layer_kinds, shared), f)
    header, blobs, off = {}, [], 0
    for name, a in named.items():
        raw = np.ascontiguousarray(a, dtype=np.uint16).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(os.path.join(directory, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for raw in blobs:
            f.write(raw)


class Gemma4Oracle:
    """Gemma4CpuDecoder (cpu/decoder.rs:27-192): prefill / advance_prefill / decode."""

    def __init__(self, cfg, weights):
        self.L = lib()
        self.cfg = cfg
        self.weights = weights
        err = ctypes.create_string_buffer(256)
        self.h = self.L.g4_open(ctypes.byref(cfg), ctypes.byref(weights), err, 256)
        if not self.h:
            raise ValueError(err.value.decode())

    def close(self):
        if self.h:
            self.L.g4_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def position(self):
        return self.L.g4_position(self.h)

    def reset(self):
        self.L.g4_reset(self.h)

    def _step(self, tokens, logits):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros(self.cfg.vocab, np.uint16) if logits else None
        rc = self.L.g4_step(self.h, ptr(t), len(t), ptr(out) if logits else None)
        if rc != 0:
            raise ValueError("empty, overlong or out-of-range token chunk")
        return out

    def prefill(self, tokens):
        return self._step(tokens, True)

    def advance_prefill(self, tokens):
        self._step(tokens, False)

    def decode(self, token):
        return self._step([token], True)

    def argmax(self, logits):
        return int(self.L.g4_argmax(ptr(logits), len(logits)))

    def generate(self, prompt, n_new):
        """Greedy continuation: prefill the prompt, then decode n_new - 1 more tokens."""
        toks = []
        lg = self.prefill(prompt)
        for i in range(n_new):
            t = self.argmax(lg)
            toks.append(t)
            if i + 1 < n_new:
                lg = self.decode(t)
        return toks
