"""Synthetic GGUF models for the decode path: the benchmark configurations and the
reference's toy fixtures.

Shapes, quant mix and workloads follow the benchmark configurations of this
build (TinyLlama-, Llama-3.1-8B- and Qwen3-8B-shaped).  Weights are seeded
N(0, 0.02), norm weights 1.0, quantized by this package's own quantizers
(synth/zs.c).  The toy fixtures restate runtime/llama_fixture.zig of the
reference (14-token vocab, identity embedding, "transition" output head).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

from . import gguf
from ._lib import synth as _synth
from .gguf import F16, F32, IQ4_XS, Q3_K, Q4_K, Q6_K, Q8_0, TensorInfo


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_seed(model_seed: int, name: str) -> int:
    return (fnv1a64(name) ^ ((model_seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def fill_tensor(dst: np.ndarray, ttype: int, rows: int, cols: int, seed: int, mean: float = 0.0,
                std: float = 0.02, threads: int | None = None) -> None:
    assert dst.dtype == np.uint8 and dst.flags["C_CONTIGUOUS"]
    need = gguf.row_bytes(ttype, cols) * rows
    if dst.nbytes < need:
        raise ValueError("destination too small")
    st = _synth().zs_fill_tensor(dst.ctypes.data, ttype, rows, cols, seed, mean, std,
                                 threads or default_threads())
    if st:
        raise RuntimeError(f"zs_fill_tensor failed ({st})")


def quantize_rows(x: np.ndarray, ttype: int) -> np.ndarray:
    """Quantizes a float32 [rows, cols] array with this package's quantizers."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, cols = x.shape
    rb = gguf.row_bytes(ttype, cols)
    out = np.zeros(rows * rb, dtype=np.uint8)
    lib = _synth()
    for r in range(rows):
        if lib.zs_quantize_row(ttype, x[r].ctypes.data, cols, out[r * rb:].ctypes.data):
            raise ValueError("quantize failed")
    return out


def normal_row(seed: int, row: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _synth().zs_normal_row(seed, row, mean, std, out.ctypes.data, n)
    return out


@dataclass
class ModelSpec:
    name: str
    arch: str  # "llama" (interleaved RoPE) or "qwen3" (NeoX RoPE)
    n_layers: int
    hidden: int
    ffn: int
    n_head: int
    n_kv: int
    head_dim: int
    vocab: int
    rope_theta: float
    eps: float
    context: int
    qk_norm: bool = False
    default_type: int = Q4_K
    attn_v_type: int = Q6_K
    output_type: int = Q6_K
    embd_type: int = Q4_K
    down_q6k_layers: set = field(default_factory=set)
    weight_std: float = 0.02

    def tensors(self) -> list:
        H, F, hd = self.hidden, self.ffn, self.head_dim
        out = [TensorInfo("token_embd.weight", self.embd_type, (H, self.vocab)),
               TensorInfo("output_norm.weight", F32, (H,)),
               TensorInfo("output.weight", self.output_type, (H, self.vocab))]
        for i in range(self.n_layers):
            p = f"blk.{i}."
            down_t = Q6_K if i in self.down_q6k_layers else self.default_type
            out += [TensorInfo(p + "attn_norm.weight", F32, (H,)),
                    TensorInfo(p + "attn_q.weight", self.default_type, (H, self.n_head * hd)),
                    TensorInfo(p + "attn_k.weight", self.default_type, (H, self.n_kv * hd)),
                    TensorInfo(p + "attn_v.weight", self.attn_v_type, (H, self.n_kv * hd)),
                    TensorInfo(p + "attn_output.weight", self.default_type, (self.n_head * hd, H)),
                    TensorInfo(p + "ffn_norm.weight", F32, (H,)),
                    TensorInfo(p + "ffn_gate.weight", self.default_type, (H, F)),
                    TensorInfo(p + "ffn_up.weight", self.default_type, (H, F)),
                    TensorInfo(p + "ffn_down.weight", down_t, (F, H))]
            if self.qk_norm:
                out += [TensorInfo(p + "attn_q_norm.weight", F32, (hd,)),
                        TensorInfo(p + "attn_k_norm.weight", F32, (hd,))]
        return out

    def metadata(self) -> list:
        a = self.arch
        md = [("general.type", gguf.T_STR, "model"),
              ("general.architecture", gguf.T_STR, a),
              ("general.alignment", gguf.T_U32, 32),
              (f"{a}.block_count", gguf.T_U32, self.n_layers),
              (f"{a}.context_length", gguf.T_U32, self.context),
              (f"{a}.embedding_length", gguf.T_U32, self.hidden),
              (f"{a}.feed_forward_length", gguf.T_U32, self.ffn),
              (f"{a}.attention.head_count", gguf.T_U32, self.n_head),
              (f"{a}.attention.head_count_kv", gguf.T_U32, self.n_kv),
              (f"{a}.attention.key_length", gguf.T_U32, self.head_dim),
              (f"{a}.attention.value_length", gguf.T_U32, self.head_dim),
              (f"{a}.rope.dimension_count", gguf.T_U32, self.head_dim),
              (f"{a}.attention.layer_norm_rms_epsilon", gguf.T_F32, self.eps),
              (f"{a}.rope.freq_base", gguf.T_F32, self.rope_theta)]
        tokens = ["<unk>", "<s>", "</s>"] + [f"<t{i}>" for i in range(3, self.vocab)]
        if a == "llama":
            md += [("tokenizer.ggml.model", gguf.T_STR, "llama"),
                   ("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_STR, tokens)),
                   ("tokenizer.ggml.scores", gguf.T_ARR, (gguf.T_F32, np.zeros(self.vocab, np.float32))),
                   ("tokenizer.ggml.token_type", gguf.T_ARR, (gguf.T_U32, np.ones(self.vocab, np.uint32)))]
        else:
            md += [("tokenizer.ggml.model", gguf.T_STR, "gpt2"),
                   ("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_STR, tokens)),
                   ("tokenizer.ggml.merges", gguf.T_ARR, (gguf.T_STR, ["< t"]))]
        md += [("tokenizer.ggml.bos_token_id", gguf.T_U32, 1),
               ("tokenizer.ggml.eos_token_id", gguf.T_U32, 2)]
        return md

    def weight_bytes_per_token(self) -> int:
        """Weight bytes one decode step streams: every projection + norms + one embedding row."""
        total = 0
        for t in self.tensors():
            if t.name == "token_embd.weight":
                total += gguf.row_bytes(t.ttype, t.row_len)
            else:
                total += t.nbytes
        return total

    def matmul_params_per_layer(self) -> int:
        """Weights one token meets in a layer's projections (q, k, v, o, gate, up, down)."""
        H, F, hd = self.hidden, self.ffn, self.head_dim
        return H * (self.n_head * hd) * 2 + H * (self.n_kv * hd) * 2 + 3 * H * F

    def prompt_pass_flops(self, tokens: int) -> int:
        """Multiply-add flops (x2) of batched prompt passes over `tokens` rows from position 0: the layer
        projections and the causal attention (scores and values), without the output head."""
        proj = 2 * tokens * self.matmul_params_per_layer()
        attn = 2 * 2 * self.n_head * self.head_dim * (tokens * (tokens + 1) // 2)
        return self.n_layers * (proj + attn)

    def kv_bytes_per_token(self, position: int) -> int:
        """fp16 K+V bytes one decode step at `position` reads (pos+1 rows) and writes (one row)."""
        kv_dim = self.n_kv * self.head_dim
        return self.n_layers * kv_dim * 2 * 2 * (position + 1) + self.n_layers * kv_dim * 2 * 2


def q6k_down_rule(i: int) -> bool:
    """Layers whose ffn_down is Q6_K in this build's Q4_K_M mix: i < 4, i >= 28 or (i - 4) % 3 == 2."""
    return i < 4 or i >= 28 or (i >= 4 and (i - 4) % 3 == 2)


def tinyllama_spec(context: int = 512) -> ModelSpec:
    return ModelSpec("tinyllama-1.1b-shaped", "llama", 22, 2048, 5632, 32, 4, 64, 32000, 10000.0, 1e-5, context,
                     down_q6k_layers={i for i in range(22) if q6k_down_rule(i)})


def llama8b_spec(context: int = 4608) -> ModelSpec:
    return ModelSpec("llama-3.1-8b-shaped", "llama", 32, 4096, 14336, 32, 8, 128, 128256, 500000.0, 1e-5, context,
                     down_q6k_layers={i for i in range(32) if q6k_down_rule(i)})


def qwen3_8b_spec(context: int = 16640) -> ModelSpec:
    return ModelSpec("qwen3-8b-shaped", "qwen3", 36, 4096, 12288, 32, 8, 128, 151936, 1000000.0, 1e-6, context,
                     qk_norm=True, default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0, embd_type=Q8_0)


def small_spec(arch: str = "llama", n_layers: int = 2, hidden: int = 256, ffn: int = 512, n_head: int = 4,
               n_kv: int = 2, head_dim: int = 64, vocab: int = 512, context: int = 128, qk_norm: bool = False,
               default_type: int = Q4_K, attn_v_type: int = Q6_K, output_type: int = Q6_K, embd_type: int = Q4_K,
               down_q6k_layers=None, rope_theta: float = 10000.0) -> ModelSpec:
    """A small model of the same structure, for parity tests the CPU oracle finishes in seconds."""
    return ModelSpec(f"small-{arch}", arch, n_layers, hidden, ffn, n_head, n_kv, head_dim, vocab, rope_theta, 1e-5,
                     context, qk_norm=qk_norm, default_type=default_type, attn_v_type=attn_v_type,
                     output_type=output_type, embd_type=embd_type,
                     down_q6k_layers=set(down_q6k_layers or ()))


def build(spec: ModelSpec, seed: int, threads: int | None = None) -> gguf.GGUFImage:
    """Lays out and fills a synthetic GGUF image for `spec`."""
    tensors = spec.tensors()
    img = gguf.layout(spec.metadata(), tensors)
    for t in tensors:
        view = img.tensor_view(t.name)
        if "_norm.weight" in t.name:
            fill_tensor(view, t.ttype, t.rows, t.row_len, 0, mean=1.0, std=0.0, threads=threads)
        else:
            fill_tensor(view, t.ttype, t.rows, t.row_len, tensor_seed(seed, t.name), std=spec.weight_std,
                        threads=threads)
    return img


def prompt_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    """Seeded uniform token ids in [3, vocab)."""
    rng = np.random.default_rng(seed)
    return rng.integers(3, vocab, size=n, dtype=np.uint32)


# ---------------- reference toy fixtures (runtime/llama_fixture.zig) ----------------

METASPACE = "▁"
TOY_VOCAB = ["<unk>", "<s>", "</s>", METASPACE + "a", METASPACE + "b", METASPACE + "c", "!", "<0xE2>", "<0x96>",
             "<0x81>", "<0x61>", "<0x62>", "<0x63>", "<0x21>"]
TOY_SCORES = [0, 0, 0, 1, 1, 1, 1, -10, -10, -10, -10, -10, -10, -10]
TOY_TYPES = [2, 3, 3, 1, 1, 1, 1, 6, 6, 6, 6, 6, 6, 6]


def _f16_bytes(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float16).view(np.uint8).ravel()


def _binary_blocks(values: np.ndarray, ttype: int, row_len: int) -> np.ndarray:
    """Binary-valued block encoders of runtime/llama_fixture.zig:342-431 (0/1 inputs only)."""
    v = np.asarray(values, dtype=np.float32).reshape(-1, row_len)
    if ttype == F32:
        return v.view(np.uint8).ravel()
    if ttype == F16:
        return _f16_bytes(v)
    if ttype in (Q3_K, IQ4_XS):  # zero blocks (:297-340)
        return np.zeros(v.shape[0] * gguf.row_bytes(ttype, row_len), dtype=np.uint8)
    nib = np.where(np.abs(v - 1) < 1e-4, 1, np.where(np.abs(v) < 1e-4, 0, -1))
    if ttype != Q8_0 and (nib < 0).any():
        raise ValueError("fixture encoders accept only 0/1 values")
    out = []
    one = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    if ttype == Q8_0:  # (:379-386): d = 1, q = +1 if v >= 0 else -1
        for row in v:
            for b in range(row_len // 32):
                blk = np.zeros(34, np.uint8)
                blk[0:2] = one
                blk[2:] = np.where(row[32 * b:32 * b + 32] >= 0, 1, 255).astype(np.uint8)
                out.append(blk)
        return np.concatenate(out)
    for r, row in enumerate(nib):
        for b in range(row_len // 256):
            q = row[256 * b:256 * b + 256].astype(np.uint8)
            if ttype == Q4_K:  # (:342-377): d=1, dmin=0, all scales 1, mins 0
                blk = np.zeros(144, np.uint8)
                blk[0:2] = one
                blk[4:8] = 1
                blk[12:16] = 1
                for g in range(4):
                    blk[16 + 32 * g:48 + 32 * g] = q[64 * g:64 * g + 32] | (q[64 * g + 32:64 * g + 64] << 4)
            elif ttype == Q6_K:  # (:388-425): qh = 0xAA, scales 1, d = 1
                blk = np.zeros(210, np.uint8)
                blk[128:192] = 0xAA
                blk[192:208] = 1
                blk[208:210] = one
                for h in range(2):
                    base = 128 * h
                    ql = blk[64 * h:64 * h + 64]
                    ql[0:32] = q[base:base + 32] | (q[base + 64:base + 96] << 4)
                    ql[32:64] = q[base + 32:base + 64] | (q[base + 96:base + 128] << 4)
            else:
                raise ValueError("unsupported fixture type")
            out.append(blk)
    return np.concatenate(out)


def toy_llama_fixture(embedding_length: int = 14, feed_forward_length: int = 4, projection_type: int = F16,
                      output_type: int = F16) -> gguf.GGUFImage:
    """makeLlamaModelFixtureWithOptions (runtime/llama_fixture.zig:66-244)."""
    embed, ff, nv = embedding_length, feed_forward_length, len(TOY_VOCAB)
    md = [("general.type", gguf.T_STR, "model"),
          ("general.architecture", gguf.T_STR, "llama"),
          ("general.alignment", gguf.T_U32, 32),
          ("tokenizer.ggml.model", gguf.T_STR, "llama"),
          ("tokenizer.ggml.tokens", gguf.T_ARR, (gguf.T_STR, TOY_VOCAB)),
          ("tokenizer.ggml.scores", gguf.T_ARR, (gguf.T_F32, TOY_SCORES)),
          ("tokenizer.ggml.token_type", gguf.T_ARR, (gguf.T_U32, TOY_TYPES)),
          ("tokenizer.ggml.bos_token_id", gguf.T_U32, 1),
          ("tokenizer.ggml.eos_token_id", gguf.T_U32, 2),
          ("tokenizer.ggml.unknown_token_id", gguf.T_U32, 0),
          ("tokenizer.ggml.add_bos_token", gguf.T_BOOL, False),
          ("tokenizer.ggml.add_eos_token", gguf.T_BOOL, False),
          ("llama.context_length", gguf.T_U32, 16),
          ("llama.embedding_length", gguf.T_U32, embed),
          ("llama.block_count", gguf.T_U32, 1),
          ("llama.feed_forward_length", gguf.T_U32, ff),
          ("llama.rope.dimension_count", gguf.T_U32, 2),
          ("llama.attention.head_count", gguf.T_U32, 1),
          ("llama.attention.head_count_kv", gguf.T_U32, 1),
          ("llama.attention.layer_norm_rms_epsilon", gguf.T_F32, 0.000001),
          ("llama.rope.freq_base", gguf.T_F32, 10000.0)]
    names = ["token_embd.weight", "output.weight", "output_norm.weight", "blk.0.attn_norm.weight",
             "blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight", "blk.0.attn_output.weight",
             "blk.0.ffn_norm.weight", "blk.0.ffn_gate.weight", "blk.0.ffn_down.weight", "blk.0.ffn_up.weight"]
    dims = [(embed, nv), (embed, nv), (embed, 1), (embed, 1), (embed, embed), (embed, embed), (embed, embed),
            (embed, embed), (embed, 1), (embed, ff), (ff, embed), (embed, ff)]
    types = [F16, output_type, F32, F32] + [projection_type] * 4 + [F32] + [projection_type] * 3
    tensors = [TensorInfo(n, t, d) for n, t, d in zip(names, types, dims)]
    img = gguf.layout(md, tensors)
    token_embd = np.zeros((nv, embed), np.float32)
    for t in range(3, nv):
        token_embd[t, t] = 1.0
    output = np.zeros((nv, embed), np.float32)
    for src, nxt in ((3, 4), (4, 5), (5, 6), (6, 3)):  # setTransition (:252-254)
        output[nxt, src] = 1.0
    ones = np.ones(embed, np.float32)
    data = [token_embd, output, ones, ones, np.zeros((embed, embed)), np.zeros((embed, embed)),
            np.zeros((embed, embed)), np.zeros((embed, embed)), ones, np.zeros((ff, embed)), np.zeros((embed, ff)),
            np.zeros((ff, embed))]
    for t, v in zip(tensors, data):
        img.tensor_view(t.name)[:] = _binary_blocks(v, t.ttype, t.row_len)
    return img


def toy_detokenize(ids) -> str:
    return "".join(TOY_VOCAB[i].replace(METASPACE, " ") for i in ids)


@dataclass
class MoeSpec:
    """A stack of Qwen3.5-MoE-style sparse FFN layers (benchmark configuration 5 at full size)."""
    name: str
    n_layers: int
    hidden: int
    n_experts: int
    top_k: int
    expert_ff: int
    shared_ff: int
    expert_type: int = IQ4_XS
    shared_type: int = Q3_K
    router_type: int = F32
    shared_gate: bool = True
    gating_func: int = 1          # softmax over all experts
    weights_norm: int = 1         # expert_weights_norm (true for qwen35moe)
    weights_scale: float = 1.0
    eps: float = 1e-6

    def weight_bytes_per_token(self) -> int:
        """Bytes one decode token streams: router (+ shared gate row), k routed experts, shared expert, norm."""
        H, F, S, k = self.hidden, self.expert_ff, self.shared_ff, self.top_k
        rb = gguf.row_bytes
        per = (rb(self.router_type, H) * (self.n_experts + (1 if self.shared_gate else 0)) + 4 * H +
               k * (2 * F * rb(self.expert_type, H) + H * rb(self.expert_type, F)) +
               (2 * S * rb(self.shared_type, H) + H * rb(self.shared_type, S) if S else 0))
        return per * self.n_layers

    def weight_bytes_all(self) -> int:
        """Bytes of every layer's weights: what one prefill pass streams when every expert is routed to."""
        H, F, S, E = self.hidden, self.expert_ff, self.shared_ff, self.n_experts
        rb = gguf.row_bytes
        per = (rb(self.router_type, H) * (E + (1 if self.shared_gate else 0)) + 4 * H +
               E * (2 * F * rb(self.expert_type, H) + H * rb(self.expert_type, F)) +
               (2 * S * rb(self.shared_type, H) + H * rb(self.shared_type, S) if S else 0))
        return per * self.n_layers

    def flops_per_token(self) -> int:
        """Multiply-adds x 2 of one token through the stack (router, k routed + shared SwiGLU experts)."""
        H, F, S, E, k = self.hidden, self.expert_ff, self.shared_ff, self.n_experts, self.top_k
        per = 2 * H * (E + (1 if self.shared_gate else 0)) + 2 * 3 * H * (k * F + S)
        return per * self.n_layers


def moe_config5_spec(n_layers: int = 40) -> MoeSpec:
    return MoeSpec("qwen3.5-moe-ffn-stack", n_layers, 2048, 256, 8, 512, 512)


def small_moe_spec(n_layers: int = 3) -> MoeSpec:
    return MoeSpec("small-moe", n_layers, 256, 16, 4, 256, 256)


def build_moe_stack(spec: MoeSpec, seed: int, threads: int | None = None):
    """Per-layer tensors {name: (bytes, rows, cols, type)}: N(0, 0.02) expert weights quantized by this
    package, router rows N(0, 1/sqrt(hidden)) so normed inputs give ~N(0, 1) logits, norm weights 1."""
    H, E, F, S = spec.hidden, spec.n_experts, spec.expert_ff, spec.shared_ff
    layers = []

    def t(name, rows, cols, ttype, std):
        buf = np.zeros(gguf.row_bytes(ttype, cols) * rows, np.uint8)
        fill_tensor(buf, ttype, rows, cols, tensor_seed(seed, name), 0.0, std, threads)
        return (buf, rows, cols, ttype)

    for i in range(spec.n_layers):
        lay = {"ffn_norm": (np.ones(H, np.float32).view(np.uint8), 1, H, F32),
               "router": t(f"blk.{i}.ffn_gate_inp", E, H, spec.router_type, H ** -0.5),
               "gate_exps": t(f"blk.{i}.ffn_gate_exps", E * F, H, spec.expert_type, 0.02),
               "up_exps": t(f"blk.{i}.ffn_up_exps", E * F, H, spec.expert_type, 0.02),
               "down_exps": t(f"blk.{i}.ffn_down_exps", E * H, F, spec.expert_type, 0.02)}
        if S:
            lay["gate_shexp"] = t(f"blk.{i}.ffn_gate_shexp", S, H, spec.shared_type, 0.02)
            lay["up_shexp"] = t(f"blk.{i}.ffn_up_shexp", S, H, spec.shared_type, 0.02)
            lay["down_shexp"] = t(f"blk.{i}.ffn_down_shexp", H, S, spec.shared_type, 0.02)
            if spec.shared_gate:
                lay["gate_inp_shexp"] = t(f"blk.{i}.ffn_gate_inp_shexp", 1, H, spec.router_type, H ** -0.5)
        layers.append(lay)
    return layers


def moe_desc(spec: MoeSpec):
    from .hip import MoeDesc
    return MoeDesc(spec.hidden, spec.n_experts, spec.top_k, spec.expert_ff, spec.shared_ff, spec.gating_func,
                   spec.weights_norm, spec.weights_scale, spec.eps)
