"""CPU checks: the C-ABI library loads and exports every declared symbol; this
build's quantizers round-trip within their format's error; the synthetic
model builder and GGUF layout are deterministic and loadable."""
import ctypes

import numpy as np
import pytest

from oracle import zo
from zhip import gguf, hip, synth
from zhip._lib import HIP_LIB
from zhip.gguf import F16, F32, IQ4_XS, Q3_K, Q4_K, Q6_K, Q8_0


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(HIP_LIB)
    names = hip.exported_symbols()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_library_reports_no_device_without_gpu():
    import os
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        pytest.skip("a GPU is visible")
    with pytest.raises(hip.HipError) as e:
        hip.Context(0)
    assert e.value.status == 1  # UNAVAILABLE, never a silent fallback


# relative RMS error bounds of one-pass quantizers on N(0, 0.02) data
BOUNDS = {Q8_0: 0.01, Q6_K: 0.03, Q4_K: 0.12, Q3_K: 0.35, IQ4_XS: 0.12, F16: 1e-3, F32: 0.0}


@pytest.mark.parametrize("ttype", list(BOUNDS))
def test_quantizer_round_trip(ttype):
    rows, cols = 16, 512
    x = np.stack([synth.normal_row(1234, r, cols, 0.0, 0.02) for r in range(rows)])
    q = synth.quantize_rows(x, ttype)
    d = zo.dequantize(ttype, q, rows, cols)
    rel = np.sqrt(np.mean((d - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel <= BOUNDS[ttype] + 1e-12, rel


def test_fill_is_deterministic_across_thread_counts():
    a = np.zeros(gguf.row_bytes(Q4_K, 1024) * 64, np.uint8)
    b = np.zeros_like(a)
    synth.fill_tensor(a, Q4_K, 64, 1024, seed=99, threads=1)
    synth.fill_tensor(b, Q4_K, 64, 1024, seed=99, threads=7)
    assert np.array_equal(a, b)


def test_synthetic_model_loads_in_oracle():
    spec = synth.small_spec()
    img = synth.build(spec, seed=5)
    m = zo.Model(img.buf)
    assert m.info.block_count == spec.n_layers and m.info.vocab_size == spec.vocab
    assert m.info.rope_style == 0
    again = synth.build(spec, seed=5)
    assert np.array_equal(img.buf, again.buf)
    r = gguf.read(img.buf)
    assert set(r.tensors) == set(img.tensors)
    assert r.data_offset == img.data_offset


def test_q4km_mix_rule_counts():
    # 16 of 32 Llama layers and 10 of 22 TinyLlama layers use Q6_K ffn_down
    assert len(synth.llama8b_spec().down_q6k_layers) == 16
    assert len(synth.tinyllama_spec().down_q6k_layers) == 10


def test_llama8b_bytes_per_token():
    spec = synth.llama8b_spec()
    assert spec.weight_bytes_per_token() + spec.kv_bytes_per_token(4095) - 32 * 1024 * 2 * 2 == \
        4_634_700_032 + 536_870_912 - 4096 * 4 * 0
