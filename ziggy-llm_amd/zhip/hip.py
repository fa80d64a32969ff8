"""ctypes binding of libziggy_hip's C ABI (include/ziggy_hip.h).

This plays the role the reference's Zig wrapper (src/runtime/metal_backend.zig)
plays for Metal: it owns handles, checks sizes, and turns status codes into
exceptions carrying the library's error message (metal_backend.zig:2027-2047).
There is no fallback: if the library is missing or no gfx950 device is
present, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import gguf
from ._lib import HIP_LIB, load

ERR_LEN = 256
STATUS = {0: "OK", 1: "UNAVAILABLE", 2: "INITIALIZATION_FAILED", 3: "COMPILATION_FAILED", 4: "BUFFER_FAILED",
          5: "EXECUTION_FAILED", 6: "INVALID_ARGUMENT"}


class HipError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("arch", ctypes.c_char * 64), ("total_memory", ctypes.c_uint64),
                ("compute_units", ctypes.c_uint32), ("wavefront_size", ctypes.c_uint32),
                ("clock_khz", ctypes.c_uint32), ("l2_bytes", ctypes.c_uint32)]


class CommitStats(ctypes.Structure):
    _fields_ = [("cpu_wait_ns", ctypes.c_uint64), ("gpu_elapsed_ns", ctypes.c_uint64),
                ("gpu_timestamps_valid", ctypes.c_bool)]


class TensorDesc(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("rows", ctypes.c_uint64), ("cols", ctypes.c_uint64),
                ("tensor_type", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


LAYER_FIELDS = ["attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "attn_q_bias", "attn_k_bias",
                "attn_v_bias", "attn_q_norm", "attn_k_norm", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down"]


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, TensorDesc) for n in LAYER_FIELDS]


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "embedding_length", "block_count", "context_length", "feed_forward_length", "head_count", "head_count_kv",
        "head_dim", "rope_dim", "vocab_size", "rope_style")] + [("rms_norm_eps", ctypes.c_float),
                                                               ("rope_freq_base", ctypes.c_float)]


class ChainProbe(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_uint64), ("kernels", ctypes.c_uint32), ("workgroups", ctypes.c_uint32),
                ("one_kernel_ms", ctypes.c_double), ("chain_ms", ctypes.c_double), ("empty_chain_ms", ctypes.c_double)]


class SyncProbe(ctypes.Structure):
    _fields_ = [("workgroups", ctypes.c_uint32), ("timed_out", ctypes.c_int32),
                ("handoff_relaxed_us", ctypes.c_double), ("handoff_acqrel_us", ctypes.c_double),
                ("barrier_flags_us", ctypes.c_double), ("barrier_counter_us", ctypes.c_double)]


class RowLoadProbe(ctypes.Structure):
    _fields_ = [("workgroups", ctypes.c_uint32), ("values", ctypes.c_uint32),
                ("slot_us", ctypes.c_double * 2), ("coalesced_us", ctypes.c_double * 2), ("lds_us", ctypes.c_double * 2)]


class GenerateStats(ctypes.Structure):
    _fields_ = [("steps", ctypes.c_uint64), ("gpu_elapsed_ns", ctypes.c_uint64), ("wall_ns", ctypes.c_uint64),
                ("next_token", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("prompt_ns", ctypes.c_uint64)]


MOE_LAYER_FIELDS = ["ffn_norm", "router", "gate_exps", "up_exps", "down_exps", "gate_shexp", "up_shexp",
                    "down_shexp", "gate_inp_shexp"]


class ShortlistEntry(ctypes.Structure):
    _fields_ = [("token_id", ctypes.c_uint32), ("logit", ctypes.c_float)]


class SamplingOptions(ctypes.Structure):
    """The sampling fields of GenerationOptions (runtime/types.zig:171-185)."""
    _fields_ = [("temperature", ctypes.c_float), ("repeat_penalty", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("top_p", ctypes.c_float), ("min_p", ctypes.c_float)]

    def __init__(self, temperature=0.0, repeat_penalty=1.0, top_k=0, top_p=1.0, min_p=0.0):
        super().__init__(temperature, repeat_penalty, top_k, top_p, min_p)


class MoeLayerDesc(ctypes.Structure):
    _fields_ = [(n, TensorDesc) for n in MOE_LAYER_FIELDS]


class MoeDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("hidden", "expert_count", "expert_used_count", "expert_ff_length",
                                               "shared_ff_length", "gating_func", "weights_norm")] + [
        ("weights_scale", ctypes.c_float), ("rms_norm_eps", ctypes.c_float)]


KERNELS = {"qkv": 0, "rope_kv": 1, "attention": 2, "o_proj": 3, "gate_up": 4, "down": 5, "output": 6,
           "qkv_attention": 7}

# the decode profiler's record kinds (ZIGGY_HIP_PROFILE_*): the reference's
# Category values (runtime/metal_profile.zig:3-27), then the calls that are not
PROFILE_CATEGORIES = ["projections", "attention", "kv_writes", "normalization", "elementwise_ops", "output_reduce",
                      "commit_wait", "host_readback", "cpu_sampling"]
PROFILE_KINDS = {**{n: k for k, n in enumerate(PROFILE_CATEGORIES)}, "commit_wait_gpu": 16, "moon_quant": 17,
                 "token_begin": 32, "token_end": 33}
PROFILE_RECORD = np.dtype([("kind", "<u4"), ("has_shape", "<u4"), ("ns", "<u8"), ("rows", "<u8"), ("cols", "<u8"),
                           ("depth", "<u8"), ("extra", "<u8"), ("tensor_type", "<u4"), ("reserved", "<u4")])
assert PROFILE_RECORD.itemsize == 56


_typed = False


def lib() -> ctypes.CDLL:
    global _typed
    L = load(HIP_LIB)
    if _typed:
        return L
    vp, sz, u32, i, f, ep = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, ctypes.c_float,
                             ctypes.c_char_p)
    E = [ep, sz]
    sigs = {
        "ziggy_hip_create_context": [i, ctypes.POINTER(vp), ctypes.POINTER(DeviceInfo)] + E,
        "ziggy_hip_destroy_context": [vp],
        "ziggy_hip_create_buffer": [vp, vp, sz, ctypes.POINTER(vp)] + E,
        "ziggy_hip_create_empty_buffer": [vp, sz, ctypes.POINTER(vp)] + E,
        "ziggy_hip_destroy_buffer": [vp],
        "ziggy_hip_buffer_length": [vp],
        "ziggy_hip_write_buffer": [vp, vp, sz, sz] + E,
        "ziggy_hip_read_buffer": [vp, vp, sz, sz] + E,
        "ziggy_hip_copy_buffer_region": [vp, vp, sz, vp, sz, sz] + E,
        "ziggy_hip_begin_sequence": [vp] + E,
        "ziggy_hip_commit_sequence": [vp] + E,
        "ziggy_hip_commit_sequence_timed": [vp, ctypes.POINTER(CommitStats)] + E,
        "ziggy_hip_run_matvec": [vp, u32, vp, sz, vp, vp, sz, u32, u32, i] + E,
        "ziggy_hip_run_matvec_silu_down_add": [vp, u32, vp, vp, vp, vp, u32, u32] + E,
        "ziggy_hip_run_matvec_argmax": [vp, u32, vp, vp, vp, u32, u32] + E,
        "ziggy_hip_dequantize_rows": [vp, u32, vp, sz, vp, u32, u32] + E,
        "ziggy_hip_time_matvec": [vp, u32, vp, u32, sz, vp, vp, u32, u32, u32, ctypes.POINTER(ctypes.c_uint64)] + E,
        "ziggy_hip_probe_chain": [vp, vp, u32, u32, ctypes.POINTER(ChainProbe)] + E,
        "ziggy_hip_probe_sync": [vp, u32, ctypes.POINTER(SyncProbe)] + E,
        "ziggy_hip_probe_row_load": [vp, u32, ctypes.POINTER(RowLoadProbe)] + E,
        "ziggy_hip_indexed_matvec": [vp, u32, vp, vp, vp, u32, u32, vp, u32, u32, i] + E,
        "ziggy_hip_run_gemm": [vp, u32, vp, vp, vp, u32, u32, u32, i] + E,
        "ziggy_hip_dual_indexed_matvec": [vp, u32, vp, vp, vp, vp, vp, u32, u32, vp, u32, u32] + E,
        "ziggy_hip_apply_rope_f32": [vp, vp, u32, u32, u32, u32, f, u32] + E,
        "ziggy_hip_apply_rope_to_dst_f32": [vp, vp, vp, sz, u32, u32, u32, u32, f, u32] + E,
        "ziggy_hip_store_kv_half": [vp, vp, vp, sz, u32] + E,
        "ziggy_hip_attention_fused_f32": [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, u32, f, f] + E,
        "ziggy_hip_attention_fused_f32_noalloc": [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, u32, f,
                                                  f] + E,
        "ziggy_hip_silu_mul_f32": [vp, vp, vp, u32] + E,
        "ziggy_hip_add_in_place_f32": [vp, vp, vp, u32] + E,
        "ziggy_hip_rms_norm_f32": [vp, vp, vp, vp, u32, f, f] + E,
        "ziggy_hip_rms_norm_per_head_f32": [vp, vp, vp, vp, u32, u32, f, f] + E,
        "ziggy_hip_argmax_f32": [vp, vp, vp, u32] + E,
        "ziggy_hip_topk_f32": [vp, vp, vp, u32, u32] + E,
        "ziggy_hip_normalize_topk_f32": [vp, vp, u32, ctypes.c_bool, ctypes.c_bool, f] + E,
        "ziggy_hip_weighted_sum_topk_f32": [vp, vp, vp, vp, u32, u32] + E,
        "ziggy_hip_sigmoid_scale_add_f32": [vp, vp, vp, vp, u32] + E,
        "ziggy_hip_session_create": [vp, ctypes.POINTER(ModelDesc), ctypes.POINTER(TensorDesc),
                                     ctypes.POINTER(TensorDesc), ctypes.POINTER(TensorDesc),
                                     ctypes.POINTER(LayerDesc), ctypes.POINTER(vp)] + E,
        "ziggy_hip_session_destroy": [vp],
        "ziggy_hip_session_reset": [vp] + E,
        "ziggy_hip_session_position": [vp],
        "ziggy_hip_session_rewind": [vp, u32] + E,
        "ziggy_hip_session_begin_token": [vp, vp] + E,
        "ziggy_hip_session_run_attention_block": [vp, u32, u32] + E,
        "ziggy_hip_session_run_ffn_block": [vp, u32] + E,
        "ziggy_hip_session_run_output": [vp, vp] + E,
        "ziggy_hip_session_run_output_argmax": [vp, ctypes.POINTER(u32)] + E,
        "ziggy_hip_session_read_hidden": [vp, vp] + E,
        "ziggy_hip_session_write_hidden": [vp, vp] + E,
        "ziggy_hip_session_read_kv": [vp, u32, u32, vp, vp] + E,
        "ziggy_hip_session_fill_kv_pattern": [vp, u32, ctypes.c_uint64] + E,
        "ziggy_hip_session_set_block_table": [vp, vp, u32] + E,
        "ziggy_hip_session_kv_pages": [vp],
        "ziggy_hip_session_step_greedy": [vp, u32, ctypes.POINTER(u32)] + E,
        "ziggy_hip_session_step_no_output": [vp, u32] + E,
        "ziggy_hip_session_generate": [vp, vp, u32, u32, vp, ctypes.POINTER(GenerateStats)] + E,
        "ziggy_hip_session_read_logits": [vp, vp] + E,
        "ziggy_hip_session_verify": [vp, u32, vp, u32, vp, ctypes.POINTER(u32)] + E,
        "ziggy_hip_session_step_shortlist": [vp, u32, u32, vp] + E,
        "ziggy_hip_session_prefill_cached": [vp, vp, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)] + E,
        "ziggy_hip_shortlist_len": [ctypes.POINTER(SamplingOptions), u32],
        "ziggy_hip_sample_shortlist": [vp, u32, vp, u32, ctypes.POINTER(SamplingOptions), ctypes.c_double,
                                       ctypes.POINTER(u32)],
        "ziggy_hip_sample_logits": [vp, u32, vp, u32, ctypes.POINTER(SamplingOptions), ctypes.c_double,
                                    ctypes.POINTER(u32)],
        "ziggy_hip_session_time_kernel": [vp, u32, u32, ctypes.POINTER(ctypes.c_uint64),
                                          ctypes.POINTER(ctypes.c_uint64)] + E,
        "ziggy_hip_profile_render": [vp, sz, vp, sz, ctypes.POINTER(sz)],
        "ziggy_hip_session_profile_decode": [vp, u32, u32, vp, vp, sz, ctypes.POINTER(sz)] + E,
        "ziggy_hip_moe_stack_create": [vp, ctypes.POINTER(MoeDesc), ctypes.POINTER(MoeLayerDesc), u32,
                                       ctypes.POINTER(vp)] + E,
        "ziggy_hip_moe_stack_destroy": [vp],
        "ziggy_hip_moe_stack_forward": [vp, vp, vp, vp, vp] + E,
        "ziggy_hip_moe_stack_time": [vp, u32, ctypes.POINTER(ctypes.c_uint64)] + E,
        "ziggy_hip_moe_stack_prefill": [vp, vp, u32, vp, vp, vp] + E,
        "ziggy_hip_moe_stack_time_prefill": [vp, u32, u32, ctypes.POINTER(ctypes.c_uint64)] + E,
        "ziggy_hip_version": [],
    }
    restypes = {"ziggy_hip_destroy_context": None, "ziggy_hip_destroy_buffer": None,
                "ziggy_hip_session_destroy": None, "ziggy_hip_moe_stack_destroy": None, "ziggy_hip_buffer_length": sz,
                "ziggy_hip_session_position": u32, "ziggy_hip_version": ctypes.c_char_p,
                "ziggy_hip_session_kv_pages": u32,
                "ziggy_hip_shortlist_len": u32}
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = restypes.get(name, i)
    _typed = True
    return L


def _call(fn_name: str, *args):
    err = ctypes.create_string_buffer(ERR_LEN)
    st = getattr(lib(), fn_name)(*args, err, ERR_LEN)
    if st:
        raise HipError(st, err.value.decode(errors="replace"))


class Buffer:
    def __init__(self, ctx: "Context", handle: ctypes.c_void_p, nbytes: int):
        self.ctx, self.h, self.nbytes = ctx, handle, nbytes

    def write(self, arr: np.ndarray, offset: int = 0):
        arr = np.ascontiguousarray(arr)
        _call("ziggy_hip_write_buffer", self.h, arr.ctypes.data, arr.nbytes, offset)

    def read(self, dtype=np.float32, count: int | None = None, offset: int = 0) -> np.ndarray:
        itemsize = np.dtype(dtype).itemsize
        n = count if count is not None else (self.nbytes - offset) // itemsize
        out = np.empty(n, dtype=dtype)
        _call("ziggy_hip_read_buffer", self.h, out.ctypes.data, out.nbytes, offset)
        return out

    def free(self):
        if self.h:
            lib().ziggy_hip_destroy_buffer(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One device context (ziggy_hip_create_context)."""

    def __init__(self, device: int = 0):
        import weakref
        h = ctypes.c_void_p()
        self.info = DeviceInfo()
        _call("ziggy_hip_create_context", device, ctypes.byref(h), ctypes.byref(self.info))
        self.h = h
        self._owned = weakref.WeakSet()  # buffers and sessions, released before the context

    def buffer(self, data: np.ndarray) -> Buffer:
        data = np.ascontiguousarray(data)
        h = ctypes.c_void_p()
        _call("ziggy_hip_create_buffer", self.h, data.ctypes.data, data.nbytes, ctypes.byref(h))
        b = Buffer(self, h, data.nbytes)
        self._owned.add(b)
        return b

    def empty(self, nbytes: int) -> Buffer:
        h = ctypes.c_void_p()
        _call("ziggy_hip_create_empty_buffer", self.h, nbytes, ctypes.byref(h))
        b = Buffer(self, h, nbytes)
        self._owned.add(b)
        return b

    # ---- primitive ops ----
    def matvec(self, ttype, m: Buffer, x: Buffer, y: Buffer, rows, cols, add=False, m_off=0, y_off=0):
        _call("ziggy_hip_run_matvec", self.h, ttype, m.h, m_off, x.h, y.h, y_off, rows, cols, int(add))

    def matvec_silu_down_add(self, ttype, m, gate, up, y, rows, cols):
        _call("ziggy_hip_run_matvec_silu_down_add", self.h, ttype, m.h, gate.h, up.h, y.h, rows, cols)

    def matvec_argmax(self, ttype, m, x, state, rows, cols):
        _call("ziggy_hip_run_matvec_argmax", self.h, ttype, m.h, x.h, state.h, rows, cols)

    def time_matvec(self, ttype, mats: Buffer, copies, copy_stride, x, y, rows, cols, iterations) -> int:
        ns = ctypes.c_uint64()
        _call("ziggy_hip_time_matvec", self.h, ttype, mats.h, copies, copy_stride, x.h, y.h, rows, cols, iterations,
              ctypes.byref(ns))
        return ns.value

    def probe_chain(self, plan, reps: int = 5) -> ChainProbe:
        """The byte plan (bytes per launch) as one kernel, as a graph of one kernel per entry, and as a
        graph of as many empty kernels (ziggy_hip_probe_chain)."""
        b = np.ascontiguousarray(plan, np.uint64)
        out = ChainProbe()
        _call("ziggy_hip_probe_chain", self.h, b.ctypes.data, b.size, reps, ctypes.byref(out))
        return out

    def probe_sync(self, rounds: int = 2000) -> SyncProbe:
        """In-launch hand-off and grid-barrier latencies (ziggy_hip_probe_sync)."""
        out = SyncProbe()
        _call("ziggy_hip_probe_sync", self.h, rounds, ctypes.byref(out))
        return out

    def probe_row_load(self, reps: int = 50) -> RowLoadProbe:
        """Per-workgroup time to bring a freshly written row into every lane, three load patterns
        (ziggy_hip_probe_row_load)."""
        out = RowLoadProbe()
        _call("ziggy_hip_probe_row_load", self.h, reps, ctypes.byref(out))
        return out

    def copy(self, src: Buffer, src_off: int, dst: Buffer, dst_off: int, nbytes: int):
        _call("ziggy_hip_copy_buffer_region", self.h, src.h, src_off, dst.h, dst_off, nbytes)

    def dequantize(self, ttype, m: Buffer, out: Buffer, rows, cols, m_off=0):
        _call("ziggy_hip_dequantize_rows", self.h, ttype, m.h, m_off, out.h, rows, cols)

    def gemm(self, ttype, m: Buffer, x: Buffer, y: Buffer, tokens: int, rows: int, cols: int, add=False):
        _call("ziggy_hip_run_gemm", self.h, ttype, m.h, x.h, y.h, tokens, rows, cols, 1 if add else 0)

    def indexed_matvec(self, ttype, m, x, y, rows, cols, entries, slot, rows_per_expert, add_weighted=False):
        _call("ziggy_hip_indexed_matvec", self.h, ttype, m.h, x.h, y.h, rows, cols, entries.h, slot,
              rows_per_expert, int(add_weighted))

    def dual_indexed_matvec(self, ttype, ma, mb, x, ya, yb, rows, cols, entries, slot, rows_per_expert):
        _call("ziggy_hip_dual_indexed_matvec", self.h, ttype, ma.h, mb.h, x.h, ya.h, yb.h, rows, cols, entries.h,
              slot, rows_per_expert)

    def rope(self, v: Buffer, heads, hd, rope_dim, pos, base, style):
        _call("ziggy_hip_apply_rope_f32", self.h, v.h, heads, hd, rope_dim, pos, base, style)

    def rope_to_dst(self, src, dst, dst_off, heads, hd, rope_dim, pos, base, style):
        _call("ziggy_hip_apply_rope_to_dst_f32", self.h, src.h, dst.h, dst_off, heads, hd, rope_dim, pos, base,
              style)

    def store_kv_half(self, src, dst, dst_off_el, count):
        _call("ziggy_hip_store_kv_half", self.h, src.h, dst.h, dst_off_el, count)

    def attention(self, q, kc, vc, out, heads, heads_kv, hd, kv_dim, ctx_len, pos, layer_base=0, window_start=0,
                  scale=None, softcap=0.0):
        scale = 1.0 / np.sqrt(hd) if scale is None else scale
        _call("ziggy_hip_attention_fused_f32", self.h, q.h, kc.h, vc.h, out.h, heads, heads_kv, hd, kv_dim, ctx_len,
              pos, layer_base, window_start, float(scale), float(softcap))

    def attention_noalloc(self, q, kc, vc, out, heads, heads_kv, hd, kv_dim, ctx_len, pos, layer_base=0,
                          window_start=0, scale=None, softcap=0.0):
        scale = 1.0 / np.sqrt(hd) if scale is None else scale
        _call("ziggy_hip_attention_fused_f32_noalloc", self.h, q.h, kc.h, vc.h, out.h, heads, heads_kv, hd, kv_dim,
              ctx_len, pos, layer_base, window_start, float(scale), float(softcap))

    def silu_mul(self, g, u, n):
        _call("ziggy_hip_silu_mul_f32", self.h, g.h, u.h, n)

    def add(self, d, s, n):
        _call("ziggy_hip_add_in_place_f32", self.h, d.h, s.h, n)

    def rms_norm(self, x, w, out, n, eps, offset=0.0):
        _call("ziggy_hip_rms_norm_f32", self.h, x.h, w.h, out.h, n, eps, offset)

    def rms_norm_per_head(self, x, w, out, heads, hd, eps, offset=0.0):
        _call("ziggy_hip_rms_norm_per_head_f32", self.h, x.h, w.h, out.h, heads, hd, eps, offset)

    def argmax(self, x, tok, n):
        _call("ziggy_hip_argmax_f32", self.h, x.h, tok.h, n)

    def topk(self, x, entries, n, k):
        _call("ziggy_hip_topk_f32", self.h, x.h, entries.h, n, k)

    def normalize_topk(self, entries, k, softmax, normalize, scale):
        _call("ziggy_hip_normalize_topk_f32", self.h, entries.h, k, bool(softmax), bool(normalize), scale)

    def weighted_sum_topk(self, d, s, entries, n, slot):
        _call("ziggy_hip_weighted_sum_topk_f32", self.h, d.h, s.h, entries.h, n, slot)

    def sigmoid_scale_add(self, d, s, scalar, n):
        _call("ziggy_hip_sigmoid_scale_add_f32", self.h, d.h, s.h, scalar.h, n)

    def begin(self):
        _call("ziggy_hip_begin_sequence", self.h)

    def commit(self) -> CommitStats:
        st = CommitStats()
        _call("ziggy_hip_commit_sequence_timed", self.h, ctypes.byref(st))
        return st

    def close(self):
        if self.h:
            for obj in list(getattr(self, "_owned", ())):
                obj.free() if isinstance(obj, Buffer) else obj.close()
            lib().ziggy_hip_destroy_context(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _desc(img: gguf.GGUFImage, name: str) -> TensorDesc:
    d = TensorDesc()
    t = img.tensors.get(name)
    if t is None:
        return d
    view = img.tensor_view(name)
    d.data = view.ctypes.data
    d.rows = t.rows
    d.cols = t.row_len
    d.tensor_type = t.ttype
    return d


def model_desc_from_gguf(img: gguf.GGUFImage, context: int | None = None) -> ModelDesc:
    """Hyperparameters as loadModel derives them (model/loader.zig:2596-2640)."""
    md = img.metadata
    arch = md["general.architecture"]

    def key(suffix, default=None):
        for k, v in md.items():
            if k.endswith(suffix):
                return v
        return default

    H = int(key(".embedding_length"))
    heads = int(key(".attention.head_count"))
    hd = int(key(".attention.key_length", H // heads))
    m = ModelDesc()
    m.embedding_length = H
    m.block_count = int(key(".block_count"))
    m.context_length = int(context if context is not None else key(".context_length"))
    m.feed_forward_length = int(key(".feed_forward_length"))
    m.head_count = heads
    m.head_count_kv = int(key(".attention.head_count_kv"))
    m.head_dim = hd
    m.rope_dim = int(key(".rope.dimension_count", hd))
    m.vocab_size = img.tensors.get("output.weight", img.tensors["token_embd.weight"]).rows
    m.rope_style = 1 if (arch.startswith("qwen") or arch.startswith("mistral")) else 0
    m.rms_norm_eps = float(key(".attention.layer_norm_rms_epsilon", 1e-6))
    m.rope_freq_base = float(key(".rope.freq_base", 10000.0))
    return m


class Session:
    """Decode session over a GGUF image resident in host memory (weights are uploaded once)."""

    def __init__(self, ctx: Context, img: gguf.GGUFImage, context: int | None = None):
        self.ctx, self.img = ctx, img
        self.md = model_desc_from_gguf(img, context)
        n = self.md.block_count
        layers = (LayerDesc * n)()
        for i in range(n):
            for f in LAYER_FIELDS:
                nm = f"blk.{i}.{f}.weight" if not f.endswith("_bias") else f"blk.{i}.{f[:-5]}.bias"
                setattr(layers[i], f, _desc(img, nm))
        out_name = "output.weight" if "output.weight" in img.tensors else "token_embd.weight"
        self._descs = (_desc(img, "token_embd.weight"), _desc(img, "output_norm.weight"), _desc(img, out_name),
                       layers)
        h = ctypes.c_void_p()
        _call("ziggy_hip_session_create", ctx.h, ctypes.byref(self.md), ctypes.byref(self._descs[0]),
              ctypes.byref(self._descs[1]), ctypes.byref(self._descs[2]), layers, ctypes.byref(h))
        self.h = h
        ctx._owned.add(self)

    @property
    def position(self) -> int:
        return int(lib().ziggy_hip_session_position(self.h))

    def reset(self):
        _call("ziggy_hip_session_reset", self.h)

    def rewind(self, position: int):
        _call("ziggy_hip_session_rewind", self.h, position)

    def step_greedy(self, token: int) -> int:
        nxt = ctypes.c_uint32()
        _call("ziggy_hip_session_step_greedy", self.h, token, ctypes.byref(nxt))
        return nxt.value

    def step_no_output(self, token: int):
        _call("ziggy_hip_session_step_no_output", self.h, token)

    def generate(self, prompt, steps: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(steps, 1), dtype=np.uint32)
        st = GenerateStats()
        _call("ziggy_hip_session_generate", self.h, prompt.ctypes.data, prompt.size, steps, out.ctypes.data,
              ctypes.byref(st))
        return out[:steps].copy(), st

    def prefill_cached(self, prompt):
        """Feeds `prompt` reusing the cached common prefix; returns (tokens reused, greedy next token)."""
        p = np.ascontiguousarray(prompt, np.uint32)
        reused, nxt = ctypes.c_uint32(), ctypes.c_uint32()
        _call("ziggy_hip_session_prefill_cached", self.h, p.ctypes.data, p.size, ctypes.byref(reused),
              ctypes.byref(nxt))
        return int(reused.value), int(nxt.value)

    def step_shortlist(self, token: int, count: int):
        """One decode step of `token`; the top-`count` logits as (token ids, logits), highest first."""
        out = (ShortlistEntry * count)()
        _call("ziggy_hip_session_step_shortlist", self.h, token, count, ctypes.cast(out, ctypes.c_void_p))
        return (np.array([e.token_id for e in out], np.uint32), np.array([e.logit for e in out], np.float32))

    def verify(self, current: int, drafts):
        """(predicted tokens [len(drafts) + 1], emitted count) of one batched verify pass."""
        drafts = np.ascontiguousarray(drafts, dtype=np.uint32)
        pred = np.zeros(drafts.size + 1, np.uint32)
        n = ctypes.c_uint32()
        _call("ziggy_hip_session_verify", self.h, current, drafts.ctypes.data if drafts.size else None,
              drafts.size, pred.ctypes.data, ctypes.byref(n))
        return pred, n.value

    def time_kernel(self, name: str, iterations: int):
        """Mean launch duration (ns) and algorithmic bytes per launch of one step kernel."""
        ns, nb = ctypes.c_uint64(), ctypes.c_uint64()
        _call("ziggy_hip_session_time_kernel", self.h, KERNELS[name], iterations, ctypes.byref(ns), ctypes.byref(nb))
        return ns.value, nb.value

    def profile_decode(self, token: int, steps: int):
        """`steps` greedy decode steps from `token`, each launch timed by HIP
        events (ziggy_hip_session_profile_decode): the greedy tokens and the
        record stream (PROFILE_RECORD), which render_profile turns into the
        reference's profile summary."""
        toks = np.zeros(steps, np.uint32)
        cap = (5 * self.md.block_count + 7) * steps
        recs = np.zeros(cap, PROFILE_RECORD)
        n = ctypes.c_size_t()
        _call("ziggy_hip_session_profile_decode", self.h, token, steps, toks.ctypes.data, recs.ctypes.data, cap,
              ctypes.byref(n))
        return toks, recs[:n.value]

    def logits(self) -> np.ndarray:
        out = np.empty(self.md.vocab_size, np.float32)
        _call("ziggy_hip_session_read_logits", self.h, out.ctypes.data)
        return out

    def kv(self, layer: int, pos: int):
        n = self.md.head_count_kv * self.md.head_dim
        k, v = np.empty(n, np.float32), np.empty(n, np.float32)
        _call("ziggy_hip_session_read_kv", self.h, layer, pos, k.ctypes.data, v.ctypes.data)
        return k, v

    @property
    def kv_pages(self) -> int:
        return int(lib().ziggy_hip_session_kv_pages(self.h))

    def set_block_table(self, table):
        """Maps logical KV page i to pool page table[i] (a permutation; on an empty cache)."""
        t = np.ascontiguousarray(table, np.uint32)
        _call("ziggy_hip_session_set_block_table", self.h, t.ctypes.data, t.size)

    def fill_kv_pattern(self, position: int, seed: int = 0):
        """The CPU oracle's deterministic K/V fill of rows [0, position); the position moves there."""
        _call("ziggy_hip_session_fill_kv_pattern", self.h, position, seed)

    # per-layer contract (gpu.Session)
    def begin_token(self, hidden: np.ndarray):
        hidden = np.ascontiguousarray(hidden, np.float32)
        _call("ziggy_hip_session_begin_token", self.h, hidden.ctypes.data)

    def run_attention_block(self, layer: int, position: int):
        _call("ziggy_hip_session_run_attention_block", self.h, layer, position)

    def run_ffn_block(self, layer: int):
        _call("ziggy_hip_session_run_ffn_block", self.h, layer)

    def run_output(self) -> np.ndarray:
        out = np.empty(self.md.vocab_size, np.float32)
        _call("ziggy_hip_session_run_output", self.h, out.ctypes.data)
        return out

    def run_output_argmax(self) -> int:
        t = ctypes.c_uint32()
        _call("ziggy_hip_session_run_output_argmax", self.h, ctypes.byref(t))
        return t.value

    def hidden(self) -> np.ndarray:
        out = np.empty(self.md.embedding_length, np.float32)
        _call("ziggy_hip_session_read_hidden", self.h, out.ctypes.data)
        return out

    def close(self):
        if getattr(self, "h", None):
            lib().ziggy_hip_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def exported_symbols() -> list:
    """Every function name declared in include/ziggy_hip.h (for ABI checks)."""
    import re
    here = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    text = open(os.path.join(here, "include", "ziggy_hip.h")).read()
    names = set(re.findall(r"\b(ziggy_hip_[a-z0-9_]+)\s*\(", text))
    for sfx in ("q4k", "q6k", "q8_0", "q3k", "f16", "dense"):
        names |= {f"ziggy_hip_run_matvec_{sfx}_f32", f"ziggy_hip_run_matvec_{sfx}_f32_to_dst",
                  f"ziggy_hip_run_matvec_{sfx}_add_f32"}
    return sorted(n for n in names if not n.endswith("_f32##") and "##" not in n)


class MoeStack:
    """A stack of MoE FFN blocks (ziggy_hip_moe_stack_*) over host-resident tensors.

    `layers` holds one dict per layer mapping MOE_LAYER_FIELDS names to
    (uint8 bytes, rows, cols, tensor type); optional tensors may be absent.
    """

    def __init__(self, ctx: Context, desc: MoeDesc, layers):
        self.ctx, self.desc, self._keep = ctx, desc, layers
        arr = (MoeLayerDesc * len(layers))()
        for i, lay in enumerate(layers):
            for f in MOE_LAYER_FIELDS:
                if f in lay:
                    data, rows, cols, ttype = lay[f]
                    setattr(arr[i], f, TensorDesc(data.ctypes.data, rows, cols, ttype, 0))
        self._arr = arr
        h = ctypes.c_void_p()
        _call("ziggy_hip_moe_stack_create", ctx.h, ctypes.byref(desc), arr, len(layers), ctypes.byref(h))
        self.h = h
        ctx._owned.add(self)

    def forward(self, hidden: np.ndarray):
        """(hidden after every layer, selected experts [layers, k], their weights)."""
        hidden = np.ascontiguousarray(hidden, np.float32)
        out = np.empty_like(hidden)
        n, k = len(self._keep), self.desc.expert_used_count
        sel = np.empty((n, k), np.uint32)
        w = np.empty((n, k), np.float32)
        _call("ziggy_hip_moe_stack_forward", self.h, hidden.ctypes.data, out.ctypes.data, sel.ctypes.data,
              w.ctypes.data)
        return out, sel, w

    def time(self, iterations: int) -> int:
        ns = ctypes.c_uint64()
        _call("ziggy_hip_moe_stack_time", self.h, iterations, ctypes.byref(ns))
        return ns.value

    def prefill(self, hidden: np.ndarray):
        """Rows [tokens][hidden] through every layer:
        (hidden rows after the stack, selected [tokens, layers, k], weights)."""
        hidden = np.ascontiguousarray(hidden, np.float32)
        assert hidden.ndim == 2 and hidden.shape[1] == self.desc.hidden
        tokens = hidden.shape[0]
        out = np.empty_like(hidden)
        n, k = len(self._keep), self.desc.expert_used_count
        sel = np.empty((tokens, n, k), np.uint32)
        w = np.empty((tokens, n, k), np.float32)
        _call("ziggy_hip_moe_stack_prefill", self.h, hidden.ctypes.data, tokens, out.ctypes.data, sel.ctypes.data,
              w.ctypes.data)
        return out, sel, w

    def time_prefill(self, tokens: int, iterations: int) -> int:
        ns = ctypes.c_uint64()
        _call("ziggy_hip_moe_stack_time_prefill", self.h, tokens, iterations, ctypes.byref(ns))
        return ns.value

    def close(self):
        if getattr(self, "h", None):
            lib().ziggy_hip_moe_stack_destroy(self.h)
            self.h = None


def render_profile(records) -> str:
    """The reference's profile summary (Profiler.renderSummary,
    runtime/metal_profile.zig:201-316) of a record stream; host code only."""
    recs = np.ascontiguousarray(records, PROFILE_RECORD)
    need = ctypes.c_size_t()
    ptr = recs.ctypes.data if recs.size else None
    st = lib().ziggy_hip_profile_render(ptr, recs.size, None, 0, ctypes.byref(need))
    if need.value == 0 and st:
        raise HipError(st, "render_profile: unknown record kind")
    buf = ctypes.create_string_buffer(need.value + 1)
    st = lib().ziggy_hip_profile_render(ptr, recs.size, buf, need.value + 1, ctypes.byref(need))
    if st:
        raise HipError(st, "render_profile: unknown record kind")
    return buf.value.decode()


def parse_profile(text: str) -> dict:
    """key=value lines of a profile summary as a dict (values as text)."""
    return dict(line.split("=", 1) for line in text.splitlines() if "=" in line)


def _sample_status(st: int, name: str):
    if st != 0:
        raise HipError(st, f"{name}: invalid arguments")


def shortlist_len(options: SamplingOptions, vocab: int) -> int:
    """shortlistLenFor (sampling.zig:47-52)."""
    return int(lib().ziggy_hip_shortlist_len(ctypes.byref(options), vocab))


def sample_shortlist(ids, logits, recent, options: SamplingOptions, uniform: float) -> int:
    """sampleShortlist (sampling.zig:31-45) on the host; uniform: the draw random.float(f64) would give."""
    n = len(ids)
    ents = (ShortlistEntry * max(n, 1))()
    for k in range(n):
        ents[k].token_id = int(ids[k])
        ents[k].logit = float(logits[k])
    rec = np.ascontiguousarray(recent, np.uint32)
    tok = ctypes.c_uint32()
    _sample_status(lib().ziggy_hip_sample_shortlist(ctypes.cast(ents, ctypes.c_void_p), n,
                                                      rec.ctypes.data if rec.size else None, rec.size,
                                                      ctypes.byref(options), uniform, ctypes.byref(tok)),
                   "sample_shortlist")
    return int(tok.value)


def sample_logits(logits, recent, options: SamplingOptions, uniform: float) -> int:
    """sampleToken (sampling.zig:11-29) on the host over full logits."""
    lg = np.ascontiguousarray(logits, np.float32)
    rec = np.ascontiguousarray(recent, np.uint32)
    tok = ctypes.c_uint32()
    _sample_status(lib().ziggy_hip_sample_logits(lg.ctypes.data, lg.size, rec.ctypes.data if rec.size else None,
                                                   rec.size, ctypes.byref(options), uniform, ctypes.byref(tok)),
                   "sample_logits")
    return int(tok.value)

