"""TIE's own call sites on the GPU: the C snippets INTEGRATION.md gives for
model_qwen3.c:404-471 (MoE branch), model_qwen3.c:390-491 (FFN half) and
model_lfm2.c:414-497 (LFM2 MoE branch), compiled against TIE's headers
(struct TIEContext, Model, LayerWeights) by oracle/Makefile into
oracle/_ref/callsite, run as a separate process on seeded inputs, and
checked against the oracle: bit for bit on the exact path (small T), within
the 16-bit bound on the matrix cores.  The binary is built where the
reference sources are and travels with the tree; without it the tests skip.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, bits, synth_layer
from oracle import bind
from tie_amd import synth

pytestmark = pytest.mark.gpu

CALLSITE = os.path.join(ROOT, "oracle", "_ref", "callsite")


def run_callsite(tmp_path, mode, layer, x, k, norm=None, eps=1e-6):
    T, d = x.shape
    with open(tmp_path / "meta.txt", "w") as f:
        f.write("%d %d %d %d %d %d %d %d %.9g\n" % (mode, d, layer.F, layer.E, k, T, layer.gate_type,
                                                   layer.down_type, eps))
    for name, a in (("router", layer.router), ("gate", layer.gate), ("up", layer.up), ("down", layer.down),
                    ("x", x)):
        np.ascontiguousarray(a).tofile(str(tmp_path / (name + ".bin")))
    if norm is not None:
        np.ascontiguousarray(norm, np.float32).tofile(str(tmp_path / "norm.bin"))
    if layer.probs_bias is not None:
        np.ascontiguousarray(layer.probs_bias, np.float32).tofile(str(tmp_path / "pbias.bin"))
    print("callsite mode %d d=%d E=%d T=%d k=%d" % (mode, d, layer.E, T, k), flush=True)
    r = subprocess.run([CALLSITE, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    return np.fromfile(str(tmp_path / "out.bin"), np.float32).reshape(T, d)


@pytest.fixture(scope="module")
def tie_table():
    if not os.path.exists(CALLSITE):
        pytest.skip("oracle/_ref/callsite not built (the reference sources were absent at build time)")
    return bind.ref_silu_table()


def test_qwen3_moe_branch_exact(tmp_path, tie_table):
    c = synth.CONFIGS["30b_t4"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None)
    x = synth.make_input(c["seed"], c["T"], c["d"])
    out = run_callsite(tmp_path, 0, layer, x, c["k"])
    ro, _, _ = bind.moe_block(layer, x, c["k"], silu_tab=tie_table)
    np.testing.assert_array_equal(bits(out), bits(ro))


def test_qwen3_moe_branch_prefill(tmp_path, tie_table):
    """T = 100: the default path at this T (the matrix cores)."""
    layer = synth_layer(301, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None)
    x = synth.make_input(301, 100, 2048)
    out = run_callsite(tmp_path, 0, layer, x, 8)
    ro, _, _ = bind.moe_block(layer, x, 8, silu_tab=tie_table)
    err = np.abs(out.astype(np.float64) - ro)
    assert err.max() <= 1e-3 * np.abs(ro).max()


def test_qwen3_ffn_half(tmp_path, tie_table):
    layer = synth_layer(302, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None)
    hidden = synth.make_input(302, 3, 2048)
    norm = synth.make_norm_weight(302, 2048)
    out = run_callsite(tmp_path, 1, layer, hidden, 8, norm=norm, eps=1e-6)
    rh, _, _ = bind.qwen3_ffn(layer, hidden, 8, norm, np.float32(1e-6), silu_tab=tie_table)
    np.testing.assert_array_equal(bits(out), bits(rh))


def test_lfm2_moe_branch(tmp_path, tie_table):
    c = synth.CONFIGS["lfm2_t32"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None, 1, c["probs_bias"])
    x = synth.make_input(c["seed"], 5, c["d"])
    out = run_callsite(tmp_path, 2, layer, x, c["k"])
    ro, _, _ = bind.moe_block(layer, x, c["k"], silu_tab=tie_table)
    np.testing.assert_array_equal(bits(out), bits(ro))
