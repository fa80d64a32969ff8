"""Pins the oracle's MoE FFN (zo_moe_ffn) against an independent float64 composition (CPU only).

The reference's MoE block is computeMoeFfn (model/loader.zig:1718-1749):
  logits = router . normed; softmax over all experts for gating 1 and 2, raw for 0 (:1722-1727);
  top-k by selectTopK (:3953-3975: descending, the lower index first among equal values);
  normalizePositiveWeights when expert_weights_norm (:3977-3990); x expert_weights_scale (:1734-1736);
  out = sum over slots of w_s * down_e(silu(gate_e . normed) * up_e . normed), expert e's gate/up rows at
        e * expert_ff and its down rows at e * hidden (computeExpertFfn :1699-1716);
  out += sigmoid(shared_gate . normed) * down_sh(silu(gate_sh . normed) * up_sh . normed)
        (computeSharedFfn :1679-1697, sigmoidScalar :4022-4029; scale 1 without the gate row).
Here that composition is written again in float64 numpy over the dequantized weights; only the block
decoders are shared with the oracle, and those are pinned bit-exactly elsewhere.  The oracle (binary32)
must agree to 1e-6 relative L2 (3e-6 at hidden 2048).  Each plausible misreading (wrong down-row offset,
the shared gate taken raw, softmax skipped, weights left unnormalised, the scale dropped) is shown to miss
by far more, so the check discriminates.
"""
import numpy as np
import pytest

from oracle import zo
from zhip import gguf, synth
from zhip.gguf import F32, IQ4_XS, Q8_0


def desc_for(spec, lay):
    def ptr(name):
        return lay[name][0].ctypes.data if name in lay else None
    return zo.MoeDesc(spec.router_type, ptr("router"), spec.expert_type, ptr("gate_exps"), ptr("up_exps"),
                      ptr("down_exps"), spec.shared_type, ptr("gate_shexp"), ptr("up_shexp"), ptr("down_shexp"),
                      spec.router_type, ptr("gate_inp_shexp"), spec.hidden, spec.expert_ff, spec.shared_ff,
                      spec.n_experts, spec.top_k, spec.gating_func, spec.weights_norm, spec.weights_scale)


def rows_f64(t, first, n):
    """Rows first .. first+n-1 of a (bytes, rows, cols, type) tensor, dequantized, as float64."""
    buf, rows, cols, ttype = t
    assert first + n <= rows
    rb = gguf.row_bytes(ttype, cols)
    if ttype == F32:
        return buf[first * rb:(first + n) * rb].view(np.float32).reshape(n, cols).astype(np.float64)
    return zo.dequantize(ttype, buf[first * rb:(first + n) * rb], n, cols).astype(np.float64)


def moe_f64(spec, lay, x, *, down_offset_ff=False, raw_shared_gate=False, skip_softmax=False, skip_norm=False,
            skip_scale=False):
    """computeMoeFfn in float64; the keyword switches plant one misreading each."""
    H, E, K, F, S = spec.hidden, spec.n_experts, spec.top_k, spec.expert_ff, spec.shared_ff
    x = x.astype(np.float64)
    logits = rows_f64(lay["router"], 0, E) @ x
    if spec.gating_func in (1, 2) and not skip_softmax:
        p = np.exp(logits - logits.max())
        logits = p / p.sum()
    order = sorted(range(E), key=lambda i: (-logits[i], i))  # descending, ties to the lower index
    sel = order[:K]
    w = logits[sel].copy()
    if spec.weights_norm and not skip_norm:
        pos = np.isfinite(w) & (w > 0)
        tot = w[pos].sum()
        w = np.where(pos, w / tot, 0.0) if tot > 0 else np.zeros_like(w)
    if spec.weights_scale != 1.0 and not skip_scale:
        w = w * spec.weights_scale

    def silu(v):
        return v / (1.0 + np.exp(-v))

    out = np.zeros(H)
    for e, ws in zip(sel, w):
        g = rows_f64(lay["gate_exps"], e * F, F) @ x
        u = rows_f64(lay["up_exps"], e * F, F) @ x
        d0 = e * F if down_offset_ff else e * H
        out += ws * (rows_f64(lay["down_exps"], d0, H) @ (silu(g) * u))
    if S:
        scale = 1.0
        if "gate_inp_shexp" in lay:
            gd = float(rows_f64(lay["gate_inp_shexp"], 0, 1)[0] @ x)
            scale = gd if raw_shared_gate else 1.0 / (1.0 + np.exp(-gd))
        g = rows_f64(lay["gate_shexp"], 0, S) @ x
        u = rows_f64(lay["up_shexp"], 0, S) @ x
        out += scale * (rows_f64(lay["down_shexp"], 0, H) @ (silu(g) * u))
    return out, np.array(sel, np.uint32), w


def rel_l2(a, b):
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-300))


CASES = {
    # softmax gating, normalised weights, gated Q3_K shared expert (the qwen35moe layout)
    "softmax-norm-shared-gate": synth.MoeSpec("pin-a", 1, 256, 16, 4, 256, 256),
    # gating_func 2 (also softmax over all experts), weights scaled, no normalisation
    "gating2-scale": synth.MoeSpec("pin-b", 1, 256, 16, 4, 256, 256, gating_func=2, weights_norm=0,
                                   weights_scale=1.5),
    # raw router logits from a Q8_0 router, scale 2, normalised
    "raw-q8-router": synth.MoeSpec("pin-c", 1, 512, 32, 8, 256, 512, router_type=Q8_0, gating_func=0,
                                   weights_norm=1, weights_scale=2.0),
    # shared expert without its gate row (scale 1)
    "shared-no-gate": synth.MoeSpec("pin-d", 1, 256, 16, 2, 256, 256, shared_gate=False),
    # no shared expert at all; one format for everything
    "no-shared": synth.MoeSpec("pin-e", 1, 256, 8, 2, 256, 0),
    "iq4-shared": synth.MoeSpec("pin-f", 1, 256, 16, 4, 256, 256, shared_type=IQ4_XS),
}


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_moe_ffn_matches_float64_composition(name):
    spec = CASES[name]
    lay = synth.build_moe_stack(spec, seed=29)[0]
    for row in range(3):
        x = zo.rms_norm(synth.normal_row(41, row, spec.hidden, 0.0, 1.0), lay["ffn_norm"][0].view(np.float32),
                        spec.eps)
        got, sel, w = zo.moe_ffn(desc_for(spec, lay), x)
        want, want_sel, want_w = moe_f64(spec, lay, x)
        assert list(sel) == list(want_sel), (name, row)
        assert np.max(np.abs(w - want_w)) <= 1e-6 * max(1.0, np.max(np.abs(want_w)))
        assert rel_l2(got, want) <= 1e-6, (name, row, rel_l2(got, want))


def test_config5_layer_shape():
    """One layer of benchmark configuration 5: hidden 2048, 256 IQ4_XS experts of FFN 512, top-8, Q3_K shared."""
    spec = synth.moe_config5_spec(1)
    lay = synth.build_moe_stack(spec, seed=3)[0]
    x = zo.rms_norm(synth.normal_row(7, 0, spec.hidden, 0.0, 1.0), lay["ffn_norm"][0].view(np.float32), spec.eps)
    got, sel, _ = zo.moe_ffn(desc_for(spec, lay), x, threads=4)
    want, want_sel, _ = moe_f64(spec, lay, x)
    assert list(sel) == list(want_sel)
    # sequential binary32 sums over 2048 terms: a few 1e-7 per dot, ~1.4e-6 here
    assert rel_l2(got, want) <= 3e-6


@pytest.mark.parametrize("plant,case", [("down_offset_ff", "raw-q8-router"),  # hidden 512 != expert_ff 256
                                        ("raw_shared_gate", "softmax-norm-shared-gate"),
                                        ("skip_softmax", "gating2-scale"),
                                        ("skip_norm", "raw-q8-router"),
                                        ("skip_scale", "gating2-scale")])
def test_planted_misreadings_are_caught(plant, case):
    """Each misreading of computeMoeFfn, planted in the float64 composition, misses the oracle by far more
    than the 1e-6 bar (or selects other experts), so the pin above tells them apart."""
    spec = CASES[case]
    lay = synth.build_moe_stack(spec, seed=29)[0]
    x = zo.rms_norm(synth.normal_row(41, 0, spec.hidden, 0.0, 1.0), lay["ffn_norm"][0].view(np.float32), spec.eps)
    got, sel, _ = zo.moe_ffn(desc_for(spec, lay), x)
    bad, bad_sel, _ = moe_f64(spec, lay, x, **{plant: True})
    assert list(bad_sel) != list(sel) or rel_l2(got, bad) > 1e-3, plant
