"""ctypes binding to the CPU oracle (oracle/build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never loads it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "build", "liboracle.so")

F32, F16, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS = 0, 1, 8, 11, 12, 13, 14, 23


class ModelInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "block_count", "embedding_length", "feed_forward_length", "context_length", "head_count", "head_count_kv",
        "key_head_dim", "value_head_dim", "rope_dim", "vocab_size", "rope_style", "expert_count",
        "expert_used_count", "expert_ff_length", "expert_gating_func", "expert_weights_norm", "has_qk_norm",
        "eos_token_id")] + [("rms_norm_eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float),
                            ("expert_weights_scale", ctypes.c_float), ("data_offset", ctypes.c_uint64)]


class MoeDesc(ctypes.Structure):
    _fields_ = [("router_type", ctypes.c_int), ("router", ctypes.c_void_p),
                ("exps_type", ctypes.c_int), ("gate_exps", ctypes.c_void_p), ("up_exps", ctypes.c_void_p),
                ("down_exps", ctypes.c_void_p),
                ("shared_type", ctypes.c_int), ("gate_sh", ctypes.c_void_p), ("up_sh", ctypes.c_void_p),
                ("down_sh", ctypes.c_void_p),
                ("shared_gate_type", ctypes.c_int), ("shared_gate", ctypes.c_void_p),
                ("hidden", ctypes.c_uint32), ("expert_ff", ctypes.c_uint32), ("shared_ff", ctypes.c_uint32),
                ("expert_count", ctypes.c_uint32), ("top_k", ctypes.c_uint32),
                ("gating_func", ctypes.c_uint32), ("weights_norm", ctypes.c_uint32),
                ("weights_scale", ctypes.c_float)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"oracle not built: run `make -C {HERE}`")
        L = ctypes.CDLL(LIB)
        vp, sz, i, u32, u64, f = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32,
                                  ctypes.c_uint64, ctypes.c_float)
        sigs = {
            "zo_f16_to_f32": ([ctypes.c_uint16], f),
            "zo_round_f16": ([f], f),
            "zo_row_bytes": ([i, sz, ctypes.POINTER(sz)], i),
            "zo_scale_min_k4": ([i, vp, vp], None),
            "zo_dequantize_row": ([i, vp, sz, vp], i),
            "zo_dot_row": ([i, vp, sz, vp, ctypes.POINTER(f)], i),
            "zo_dot_simd": ([vp, vp, sz], f),
            "zo_rms_norm": ([vp, vp, vp, sz, f, f], None),
            "zo_rms_norm_per_head": ([vp, vp, vp, sz, sz, f, f], None),
            "zo_apply_rope": ([vp, sz, sz, sz, sz, f, i], None),
            "zo_softmax": ([vp, sz], None),
            "zo_argmax": ([vp, sz], u32),
            "zo_silu_in_place": ([vp, sz], None),
            "zo_sigmoid": ([f], f),
            "zo_select_topk": ([vp, sz, vp, vp, sz], None),
            "zo_normalize_positive": ([vp, sz], None),
            "zo_attention": ([vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, vp], None),
            "zo_matvec": ([i, vp, sz, sz, vp, vp, i], i),
            "zo_model_open": ([vp, sz, ctypes.POINTER(vp)], i),
            "zo_model_close": ([vp], None),
            "zo_model_get_info": ([vp, ctypes.POINTER(ModelInfo)], i),
            "zo_model_tensor": ([vp, ctypes.c_char_p, ctypes.POINTER(u32), ctypes.POINTER(u64),
                                 ctypes.POINTER(u64), ctypes.POINTER(u64)], i),
            "zo_session_create": ([vp, u32, i, i, ctypes.POINTER(vp)], i),
            "zo_session_destroy": ([vp], None),
            "zo_session_reset": ([vp], None),
            "zo_session_position": ([vp], u32),
            "zo_session_set_position": ([vp, u32], i),
            "zo_session_step": ([vp, u32, vp], i),
            "zo_session_step_greedy": ([vp, u32, ctypes.POINTER(u32)], i),
            "zo_session_step_no_output": ([vp, u32], i),
            "zo_session_hidden": ([vp, vp], i),
            "zo_session_kv": ([vp, u32, u32, vp, vp], i),
            "zo_session_fill_kv_pattern": ([vp, u32, u64], i),
            "zo_generate": ([vp, vp, sz, sz, i, vp, ctypes.POINTER(sz), ctypes.POINTER(u64)], i),
            "zo_moe_ffn": ([ctypes.POINTER(MoeDesc), vp, vp, vp, vp, i], i),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _check(st: int, what: str) -> None:
    if st:
        raise RuntimeError(f"oracle {what} failed with status {st}")


def round_f16(values) -> np.ndarray:
    """zo_round_f16 over an array: f32 -> binary16 -> f32 as the f16 KV cache stores it."""
    v = np.ascontiguousarray(values, np.float32).ravel()
    f = lib().zo_round_f16
    return np.array([f(float(x)) for x in v], np.float32)


def row_bytes(ttype: int, cols: int) -> int:
    out = ctypes.c_size_t()
    _check(lib().zo_row_bytes(ttype, cols, ctypes.byref(out)), "row_bytes")
    return out.value


def dequantize(ttype: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    rb = row_bytes(ttype, cols)
    out = np.empty((rows, cols), np.float32)
    for r in range(rows):
        _check(lib().zo_dequantize_row(ttype, data[r * rb:].ctypes.data, cols, out[r].ctypes.data), "dequantize")
    return out


def dot_row(ttype: int, row: np.ndarray, x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, np.float32)
    row = np.ascontiguousarray(row, np.uint8)
    out = ctypes.c_float()
    _check(lib().zo_dot_row(ttype, _ptr(row), x.size, _ptr(x), ctypes.byref(out)), "dot_row")
    return out.value


def matvec(ttype: int, data: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check(lib().zo_matvec(ttype, _ptr(data), rows, cols, _ptr(x), _ptr(y), threads), "matvec")
    return y


def rms_norm(x, w, eps, offset=0.0):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().zo_rms_norm(_ptr(out), _ptr(x), _ptr(w), x.size, eps, offset)
    return out


def rms_norm_per_head(x, w, head_count, head_dim, eps, offset=0.0):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().zo_rms_norm_per_head(_ptr(out), _ptr(x), _ptr(w), head_count, head_dim, eps, offset)
    return out


def rope(v, head_count, head_dim, rope_dim, position, base, style):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().zo_apply_rope(_ptr(v), head_count, head_dim, rope_dim, position, base, style)
    return v


def attention(q, k_cache, v_cache, head_count, head_count_kv, head_dim, position, window_start=0):
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(k_cache, np.float32)
    vc = np.ascontiguousarray(v_cache, np.float32)
    out = np.empty(head_count * head_dim, np.float32)
    scores = np.empty(position + 1, np.float32)
    lib().zo_attention(_ptr(out), _ptr(q), _ptr(kc), _ptr(vc), head_count, head_count_kv, head_dim,
                       head_count_kv * head_dim, position, window_start, _ptr(scores))
    return out


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().zo_argmax(_ptr(v), v.size))


def select_topk(probs, k):
    probs = np.ascontiguousarray(probs, np.float32)
    idx = np.empty(k, np.uint32)
    w = np.empty(k, np.float32)
    lib().zo_select_topk(_ptr(probs), probs.size, _ptr(idx), _ptr(w), k)
    return idx, w


def normalize_positive(w):
    w = np.array(w, dtype=np.float32, copy=True)
    lib().zo_normalize_positive(_ptr(w), w.size)
    return w


def softmax(v):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().zo_softmax(_ptr(v), v.size)
    return v


def silu(v):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().zo_silu_in_place(_ptr(v), v.size)
    return v


def scale_min_k4(j: int, scales: bytes):
    s = np.frombuffer(bytes(scales), np.uint8).copy()
    out = np.zeros(2, np.uint8)
    lib().zo_scale_min_k4(j, _ptr(s), _ptr(out))
    return int(out[0]), int(out[1])


def moe_ffn(desc: MoeDesc, normed: np.ndarray, threads: int = 1):
    normed = np.ascontiguousarray(normed, np.float32)
    out = np.empty(desc.hidden, np.float32)
    sel = np.empty(desc.top_k, np.uint32)
    selw = np.empty(desc.top_k, np.float32)
    _check(lib().zo_moe_ffn(ctypes.byref(desc), _ptr(normed), _ptr(out), _ptr(sel), _ptr(selw), threads), "moe")
    return out, sel, selw


class Model:
    """A GGUF image parsed by the oracle (model/loader.zig:2525-2785)."""

    def __init__(self, buf: np.ndarray):
        self.buf = buf  # keep alive
        h = ctypes.c_void_p()
        _check(lib().zo_model_open(buf.ctypes.data, buf.nbytes, ctypes.byref(h)), "model_open")
        self.h = h
        self.info = ModelInfo()
        lib().zo_model_get_info(h, ctypes.byref(self.info))

    def tensor(self, name: str):
        t, rl, rows, off = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().zo_model_tensor(self.h, name.encode(), ctypes.byref(t), ctypes.byref(rl), ctypes.byref(rows),
                                     ctypes.byref(off)), f"tensor {name}")
        return t.value, rl.value, rows.value, off.value

    def close(self):
        if self.h:
            lib().zo_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    """Session on the CPU path (model/loader.zig:871-1440)."""

    def __init__(self, model: Model, context: int = 0, kv_f16: bool = False, threads: int = 1):
        self.model = model
        h = ctypes.c_void_p()
        _check(lib().zo_session_create(model.h, context, int(kv_f16), threads, ctypes.byref(h)), "session_create")
        self.h = h

    @property
    def position(self) -> int:
        return int(lib().zo_session_position(self.h))

    def set_position(self, p: int):
        _check(lib().zo_session_set_position(self.h, p), "set_position")

    def reset(self):
        lib().zo_session_reset(self.h)

    def step(self, token: int) -> np.ndarray:
        logits = np.empty(self.model.info.vocab_size, np.float32)
        _check(lib().zo_session_step(self.h, token, _ptr(logits)), "step")
        return logits

    def step_greedy(self, token: int) -> int:
        nxt = ctypes.c_uint32()
        _check(lib().zo_session_step_greedy(self.h, token, ctypes.byref(nxt)), "step_greedy")
        return nxt.value

    def step_no_output(self, token: int):
        _check(lib().zo_session_step_no_output(self.h, token), "step_no_output")

    def hidden(self) -> np.ndarray:
        out = np.empty(self.model.info.embedding_length, np.float32)
        lib().zo_session_hidden(self.h, _ptr(out))
        return out

    def kv(self, layer: int, pos: int):
        n = self.model.info.head_count_kv * self.model.info.key_head_dim
        k, v = np.empty(n, np.float32), np.empty(n, np.float32)
        _check(lib().zo_session_kv(self.h, layer, pos, _ptr(k), _ptr(v)), "kv")
        return k, v

    def fill_kv_pattern(self, position: int, seed: int = 0):
        _check(lib().zo_session_fill_kv_pattern(self.h, position, seed), "fill_kv_pattern")

    def generate(self, prompt, steps: int, ignore_eos: bool = True):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(steps, 1), np.uint32)
        n, ns = ctypes.c_size_t(), ctypes.c_uint64()
        _check(lib().zo_generate(self.h, _ptr(prompt), prompt.size, steps, int(ignore_eos), _ptr(out),
                                 ctypes.byref(n), ctypes.byref(ns)), "generate")
        return out[:n.value].copy(), ns.value

    def close(self):
        if self.h:
            lib().zo_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
