"""The paged binary16 KV cache: a shuffled block table gives the same results as pages in order.

The session's cache is a pool of 64-position pages per layer addressed through a block table.  Every
kernel that touches the cache goes through the table: the fused decode attention (its K/V store and
tile loads), the batched prompt passes (their K/V stores and multi-query attention) and the verify pass.
With the table a random permutation, the token stream and the logits must be bit-identical to a session
whose pages are in order (same arithmetic, other addresses; the prompt passes are deterministic) and the stream must equal the oracle's
(which keeps one contiguous cache, as the reference does: runtime/gpu/session.zig:106-111).  The cache
rows read back through the table must equal the in-order session's.  The long-position steps of
tests/test_gpu_headline.py run over a shuffled table at the Llama-3.1-8B shape.
"""
import sys

import numpy as np
import pytest

from oracle import zo
from zhip import hip, synth
from zhip.gguf import Q8_0

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


MODELS = {
    "llama-q4km-g2": dict(arch="llama", down_q6k_layers=[1], context=512),
    "qwen3-q8-g4-hd128": dict(arch="qwen3", qk_norm=True, hidden=512, ffn=1024, n_head=4, n_kv=1, head_dim=128,
                              default_type=Q8_0, attn_v_type=Q8_0, output_type=Q8_0, embd_type=Q8_0, context=512,
                              rope_theta=1000000.0),
}


@pytest.mark.parametrize("name", list(MODELS))
def test_shuffled_block_table_is_bit_identical(hip_ctx, name):
    say(f"paged kv {name}")
    spec = synth.small_spec(**MODELS[name])
    img = synth.build(spec, seed=71)
    prompt = synth.prompt_tokens(72, 300, spec.vocab)
    want, _ = zo.Session(zo.Model(img.buf), context=spec.context, kv_f16=True).generate(prompt, 64)
    a = hip.Session(hip_ctx, img, context=spec.context)
    b = hip.Session(hip_ctx, img, context=spec.context)
    assert a.kv_pages == b.kv_pages == (spec.context + 63) // 64
    table = np.random.default_rng(5).permutation(b.kv_pages).astype(np.uint32)
    assert not np.array_equal(table, np.arange(b.kv_pages))
    b.set_block_table(table)
    ga, _ = a.generate(prompt, 64)
    gb, _ = b.generate(prompt, 64)
    assert [int(t) for t in ga] == [int(t) for t in gb] == [int(t) for t in want]
    assert np.array_equal(a.logits(), b.logits())
    for layer in range(spec.n_layers):
        for pos in (0, 63, 64, 200, 299, 363):
            ka, va = a.kv(layer, pos)
            kb, vb = b.kv(layer, pos)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), (layer, pos)
    # a verify pass over the shuffled pages (multi-query attention, K/V rows stored through the table);
    # its split products add in any order, so only the predictions are compared
    cur = int(gb[-1])
    pa, na = a.verify(cur, [3, 4, 5])
    pb, nb = b.verify(cur, [3, 4, 5])
    assert na == nb and np.array_equal(pa, pb)
    a.close()
    b.close()


def test_block_table_rejects_bad_tables(hip_ctx):
    spec = synth.small_spec(context=256)
    img = synth.build(spec, seed=73)
    s = hip.Session(hip_ctx, img, context=256)
    n = s.kv_pages
    with pytest.raises(hip.HipError):
        s.set_block_table(np.arange(n - 1, dtype=np.uint32))  # wrong length
    with pytest.raises(hip.HipError):
        s.set_block_table(np.zeros(n, np.uint32))  # not a permutation
    with pytest.raises(hip.HipError):
        s.set_block_table(np.full(n, n, np.uint32))  # out of range
    s.generate(np.array([3, 4], np.uint32), 1)
    with pytest.raises(hip.HipError):
        s.set_block_table(np.arange(n, dtype=np.uint32)[::-1].copy())  # cache not empty
    s.close()
