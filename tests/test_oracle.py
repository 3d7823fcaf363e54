"""The CPU oracle (oracle/tie_oracle.c) pinned against the compiled reference's
golden vectors (tests/golden/) and against closed forms."""
import os

import numpy as np
import pytest

from conftest import bits, golden_layer, host_cpu_identity, load_golden
from oracle import bind
from tie_amd import synth

CASES = ["g30b_q4k_t4", "g235b_e16_t2", "gtiny_q4k_t8", "gtiny_q6k_q4k_t8", "gtiny_ties_t6", "g30b_bf16_zipf_t4",
         "g30b_bf16_zipf_literal_t4"]


def test_silu_table_matches_reference_build():
    g = load_golden("silu_table")
    if str(g["cpu"]) != host_cpu_identity():
        pytest.skip("golden SiLU table was built on %s; this host is %s" % (g["cpu"], host_cpu_identity()))
    np.testing.assert_array_equal(bits(bind.silu_table()), bits(g["table"]))


def test_silu_table_modes_differ_only_in_reciprocal():
    # TIE's table approximates SiLU only loosely (expf_fast is a coarse
    # Schraudolph exponential: |error| < 0.05 over [-10, 10]); the two
    # reciprocal flavours agree to a few ulp but need not agree bitwise
    t1 = bind.silu_table(1)
    xs = -10.0 + 20.0 * np.arange(8192, dtype=np.float64) / 8191.0
    ref = xs / (1.0 + np.exp(-xs))
    assert np.max(np.abs(t1 - ref)) < 0.05
    assert np.max(np.abs(t1 - ref)[xs > 5]) < 2e-3
    if bind.oracle().orc_silu_rcp_mode() == 2:
        t2 = bind.silu_table(2)
        assert np.max(np.abs(t2 - t1) / np.maximum(np.abs(t1), 1e-30)) < 1e-5


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_reference_golden(name):
    g = load_golden(name)
    layer = golden_layer(g)
    assert layer.digest() == str(g["digest"]), "synthetic generator changed"
    out, idx, w, logits = bind.moe_block(layer, g["x"], int(g["k"]), literal_bf16_stride=bool(g["literal"]),
                                         with_logits=True)
    # routing does not depend on the host's SiLU table
    np.testing.assert_array_equal(bits(logits), bits(g["logits"]))
    np.testing.assert_array_equal(idx, g["topk_idx"])
    np.testing.assert_array_equal(bits(w), bits(g["topk_w"]))
    if str(g["cpu"]) != host_cpu_identity():
        pytest.skip("outputs depend on the SiLU table of %s" % g["cpu"])
    np.testing.assert_array_equal(bits(out), bits(g["out"]))


@pytest.mark.skipif(not bind.ref_available(), reason="reference build absent")
@pytest.mark.parametrize("seed", [11, 12])
def test_oracle_matches_reference_fresh_inputs(seed):
    layer = synth.make_layer(seed, 512, 256, 32, synth.Q4_K, synth.Q6_K)
    x = synth.make_input(seed, 5, 512)
    x[2, :17] = 0.0  # zeros and a negative zero
    x[3, 5] = -0.0
    a = bind.moe_block(layer, x, 6, with_logits=True)
    b = bind.ref_moe_block(layer, x, 6, with_logits=True)
    for p, q in zip(a, b):
        np.testing.assert_array_equal(bits(p), bits(q))


def near_tie_tokens(sel_scores, k):
    """Tokens whose k-th and (k+1)-th selection scores differ by less than
    1e-5 (the tolerance band of the selection parity)."""
    s = -np.sort(-sel_scores.astype(np.float64), axis=1)
    if s.shape[1] <= k:
        return np.zeros(s.shape[0], bool)
    return np.abs(s[:, k - 1] - s[:, k]) < 1e-5


def assert_lfm2_close(a, b, k, sel_scores, what):
    """LFM2 parity bar: the oracle computes the sigmoid with scalar libm
    expf and IEEE division, TIE's compiled loop with the vectorised expf of
    -ffast-math.  Selection equal except near-tie tokens (reported), gate
    weights within 1e-6 relative, outputs within 1e-6 of max|out|."""
    (oa, ia, wa), (ob, ib, wb) = a[:3], b[:3]
    tie = near_tie_tokens(sel_scores, k)
    print("%s: %d near-tie token(s) of %d" % (what, int(tie.sum()), len(tie)))
    np.testing.assert_array_equal(ia[~tie], ib[~tie])
    np.testing.assert_allclose(wa[~tie], wb[~tie], rtol=1e-6, atol=0)
    ok = ~tie
    scale = float(np.abs(ob[ok]).max()) if ok.any() else 1.0
    err = float(np.abs(oa[ok] - ob[ok]).max()) if ok.any() else 0.0
    rel_l2 = float(np.linalg.norm(oa[ok] - ob[ok]) / max(np.linalg.norm(ob[ok]), 1e-30)) if ok.any() else 0.0
    print("%s: max|diff| %.3g of max|out| %.3g, rel L2 %.3g" % (what, err, scale, rel_l2))
    assert err <= 1e-6 * scale


def lfm2_selection_scores(layer, logits):
    p = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    return p + (layer.probs_bias if layer.probs_bias is not None else 0.0)


@pytest.mark.parametrize("name", ["glfm2_t4", "glfm2_sat_t6"])
def test_lfm2_oracle_matches_reference_golden(name):
    g = load_golden(name)
    layer = golden_layer(g)
    assert layer.digest() == str(g["digest"]), "synthetic generator changed"
    k = int(g["k"])
    res = bind.moe_block(layer, g["x"], k, with_logits=True)
    np.testing.assert_array_equal(bits(res[3]), bits(g["logits"]))
    if str(g["cpu"]) != host_cpu_identity():
        # outputs depend on the host's SiLU table; selection and weights do not
        tie = near_tie_tokens(lfm2_selection_scores(layer, g["logits"]), k)
        np.testing.assert_array_equal(res[1][~tie], g["topk_idx"][~tie])
        np.testing.assert_allclose(res[2][~tie], g["topk_w"][~tie], rtol=1e-6, atol=0)
        pytest.skip("outputs depend on the SiLU table of %s" % g["cpu"])
    assert_lfm2_close(res, (g["out"], g["topk_idx"], g["topk_w"]), k,
                      lfm2_selection_scores(layer, g["logits"]), name)


@pytest.mark.skipif(not bind.ref_available(), reason="reference build absent")
@pytest.mark.parametrize("seed,pb", [(13, 0.05), (14, None)])
def test_lfm2_oracle_matches_reference_fresh_inputs(seed, pb):
    layer = synth.make_layer(seed, 512, 512, 32, synth.Q4_K, synth.Q6_K, routing=1, probs_bias=pb)
    x = synth.make_input(seed, 24, 512)
    a = bind.moe_block(layer, x, 4, with_logits=True)
    b = bind.ref_moe_block(layer, x, 4, with_logits=True)
    np.testing.assert_array_equal(bits(a[3]), bits(b[3]))
    assert_lfm2_close(a, b, 4, lfm2_selection_scores(layer, a[3]), "lfm2 seed %d" % seed)


@pytest.mark.parametrize("seed", range(10))
def test_sigmoid_route_closed_form(seed):
    """orc_sigmoid_route against float64: selection = stable descending sort
    of sigmoid + bias (away from near ties), weights = p / (sum p + 1e-6),
    and saturated logits tie at p = 1 and fall back to the index order."""
    rng = np.random.default_rng(100 + seed)
    E = int(rng.integers(4, 160))
    k = int(rng.integers(1, min(E, 16) + 1))
    logits = rng.normal(0, 3, size=E).astype(np.float32)
    logits[rng.integers(0, E, 3)] = 40.0  # sigmoid(40) == 1.0f
    bias = rng.normal(0, 0.05, size=E).astype(np.float32) if seed % 2 else None
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    bind.oracle().orc_sigmoid_route(logits.ctypes.data, E, k, None if bias is None else bias.ctypes.data,
                                    idx.ctypes.data, w.ctypes.data)
    p32 = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    sel = p32 + (bias if bias is not None else np.float32(0.0))
    order = sorted(range(E), key=lambda e: (-float(sel[e]), e))
    # a float64 sigmoid can differ from libm's expf by an ulp: compare the
    # order where no two of the top k+1 scores are within 1e-6 (exact ties,
    # such as the saturated p = 1, are computed exactly by both)
    gap = np.abs(np.diff(-np.sort(-sel.astype(np.float64))))[:k]
    if not ((gap > 0) & (gap < 1e-6)).any():
        assert list(idx) == order[:k]
    p = p32[idx].astype(np.float64)
    np.testing.assert_allclose(w, p / (p.sum() + 1e-6), rtol=1e-6)
    assert abs(float(w.astype(np.float64).sum()) - p.sum() / (p.sum() + 1e-6)) < 1e-6


@pytest.mark.skipif(not bind.ref_available(), reason="reference build absent")
@pytest.mark.parametrize("d", [8, 256, 2048, 4104])
def test_rms_norm_matches_reference(d):
    """orc_rms_norm against the compiled rms_norm_f32_f32_f32_avx2 (through
    TIE's dispatch_rms_norm), bit for bit: rows of very different scales,
    a zero row, and a length with a tail past the 8-lane loop."""
    rng = np.random.default_rng(d)
    x = rng.normal(0, 1, size=(12, d)).astype(np.float32)
    x[1] *= np.float32(1e-4)
    x[2] *= np.float32(1e5)
    x[3] = 0.0
    w = rng.normal(1, 0.1, size=d).astype(np.float32)
    for eps in (1e-6, 1e-5):
        np.testing.assert_array_equal(bits(bind.rms_norm(x, w, eps)), bits(bind.ref_rms_norm(x, w, eps)))


def test_rms_norm_closed_form():
    """x * w / sqrt(mean(x^2) + eps) in fp64: the host's approximate
    reciprocal square root plus one Newton step is good to ~1e-7."""
    rng = np.random.default_rng(5)
    x = rng.normal(0, 2, size=(20, 2048)).astype(np.float32)
    w = rng.normal(1, 0.1, size=2048).astype(np.float32)
    got = bind.rms_norm(x, w, 1e-6).astype(np.float64)
    x64 = x.astype(np.float64)
    want = x64 * w / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=0)


@pytest.mark.parametrize("name", ["gffn_qwen3_t3", "gffn_tiny_t5"])
def test_qwen3_ffn_oracle_matches_reference_golden(name):
    """RMSNorm + block + residual against the compiled reference's vectors.
    The RMSNorm uses the host's RSQRTSS and the block the host's SiLU
    table, so the bits are compared on the CPU they were made on."""
    g = load_golden(name)
    layer = golden_layer(g)
    assert layer.digest() == str(g["digest"]), "synthetic generator changed"
    h, idx, w = bind.qwen3_ffn(layer, g["hidden"], int(g["k"]), g["ffn_norm"], float(g["eps"]))
    if str(g["cpu"]) != host_cpu_identity():
        normed = bind.rms_norm(g["hidden"], g["ffn_norm"], float(g["eps"]))
        np.testing.assert_allclose(normed, g["normed"], rtol=1e-6, atol=0)
        pytest.skip("bits depend on the RSQRTSS/SiLU of %s" % g["cpu"])
    np.testing.assert_array_equal(bits(bind.rms_norm(g["hidden"], g["ffn_norm"], float(g["eps"]))),
                                  bits(g["normed"]))
    np.testing.assert_array_equal(idx, g["topk_idx"])
    np.testing.assert_array_equal(bits(w), bits(g["topk_w"]))
    np.testing.assert_array_equal(bits(h), bits(g["hidden_out"]))


# ---------------------------------------------------------------- closed forms
def test_fp16_conversion_all_values():
    h = np.arange(65536, dtype=np.uint32)
    o = bind.oracle()
    got = np.array([o.orc_fp16_to_fp32(int(v)) for v in h[::7]], np.float32)
    want = h[::7].astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(bits(got[~nan]), bits(want[~nan]))


def _q4k_known_block():
    """d = 1, dmin = 0.5, scale_j = j + 1, min_j = 2j, quants q[i] = i % 16."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
    sc = [j + 1 for j in range(8)]
    mn = [2 * j for j in range(8)]
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    blk[4:16] = s
    qv = np.arange(256) % 16
    # sub-block 2g = low nibbles of bytes 32g..32g+31, 2g+1 = their high nibbles
    for g in range(4):
        lo = qv[64 * g:64 * g + 32]
        hi = qv[64 * g + 32:64 * g + 64]
        blk[16 + 32 * g:16 + 32 * g + 32] = (lo | (hi << 4)).astype(np.uint8)
    want = np.array([1.0 * sc[i // 32] * qv[i] - 0.5 * mn[i // 32] for i in range(256)], np.float32)
    return blk, want


def test_q4k_known_answer():
    blk, want = _q4k_known_block()
    y = np.empty(256, np.float32)
    bind.oracle().orc_dequant_q4k(blk.ctypes.data, 256, y.ctypes.data)
    np.testing.assert_array_equal(y, want)
    x = np.ones(256, np.float32)
    got = bind.oracle().orc_dot_q4k_block(x.ctypes.data, blk.ctypes.data)
    assert got == pytest.approx(float(want.astype(np.float64).sum()), rel=1e-6)


def test_q6k_known_answer():
    blk = np.zeros(210, np.uint8)
    q = (np.arange(256) * 5) % 64  # 6-bit quants
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * h + l + 32 * i] for i in range(4))
            ql[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[64 * h + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    sc = np.arange(-8, 8, dtype=np.int8)
    blk[0:128] = ql
    blk[128:192] = qh
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = np.array([0.25], np.float16).view(np.uint8)
    want = np.array([0.25 * sc[i // 16] * (q[i] - 32) for i in range(256)], np.float32)
    y = np.empty(256, np.float32)
    bind.oracle().orc_dequant_q6k(blk.ctypes.data, 256, y.ctypes.data)
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("wtype", [synth.Q4_K, synth.Q6_K])
def test_block_dot_against_fp64_dequant(wtype):
    rng = np.random.default_rng(5)
    blocks = (synth.q4k_blocks if wtype == synth.Q4_K else synth.q6k_blocks)(rng, 64)
    x = rng.normal(size=256).astype(np.float32)
    o = bind.oracle()
    for blk in blocks:
        blk = np.ascontiguousarray(blk)
        y = np.empty(256, np.float32)
        (o.orc_dequant_q4k if wtype == synth.Q4_K else o.orc_dequant_q6k)(blk.ctypes.data, 256, y.ctypes.data)
        exact = float(np.dot(y.astype(np.float64), x.astype(np.float64)))
        scale = float(np.dot(np.abs(y).astype(np.float64), np.abs(x).astype(np.float64)))
        dot = (o.orc_dot_q4k_block if wtype == synth.Q4_K else o.orc_dot_q6k_block)(x.ctypes.data, blk.ctypes.data)
        assert abs(dot - exact) <= 1e-6 * scale + 1e-30


def test_router_row_against_fp64():
    rng = np.random.default_rng(3)
    x = rng.normal(size=2048).astype(np.float32)
    w = rng.normal(0, 0.02, size=2048).astype(np.float32)
    got = bind.oracle().orc_dot_f32(x.ctypes.data, w.ctypes.data, 2048)
    exact = float(np.dot(x.astype(np.float64), w.astype(np.float64)))
    assert abs(got - exact) <= 1e-6 * float(np.abs(x * w).sum())


def _topk(logits, k):
    idx = np.empty(k, np.int32)
    sc = np.empty(k, np.float32)
    bind.oracle().orc_find_top_k(logits.ctypes.data, logits.size, k, idx.ctypes.data, sc.ctypes.data)
    return idx, sc


@pytest.mark.parametrize("seed", range(20))
def test_topk_is_stable_descending_selection(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(4, 200))
    k = int(rng.integers(1, min(E, 32) + 1))
    logits = rng.integers(-5, 5, size=E).astype(np.float32)  # many ties
    if seed % 3 == 0:
        logits[rng.integers(0, E, 3)] = np.nan
    if seed % 4 == 0:
        logits[rng.integers(0, E, 2)] = -np.inf
    idx, sc = _topk(logits, k)
    valid = [e for e in range(E) if logits[e] > -np.inf]
    order = sorted(valid, key=lambda e: (-float(logits[e]), e))[:k]
    want = order + [-1] * (k - len(order))
    assert list(idx) == want


def test_softmax_identities():
    rng = np.random.default_rng(4)
    for _ in range(50):
        v = np.sort(rng.normal(size=8).astype(np.float32))[::-1].copy()
        s = v.copy()
        bind.oracle().orc_softmax(s.ctypes.data, 8)
        assert abs(float(s.astype(np.float64).sum()) - 1.0) < 4e-7
        ref = np.exp(v.astype(np.float64) - v[0])
        ref /= ref.sum()
        np.testing.assert_allclose(s, ref, rtol=2e-6)


def test_swiglu_interpolates_and_extrapolates():
    tab = bind.silu_table()
    x = np.array([-30.0, -10.5, -3.3, -0.01, 0.0, 0.7, 5.5, 9.99, 12.0, 200.0], np.float32)
    up = np.full_like(x, 2.0)
    g = x.copy()
    bind.oracle().orc_swiglu(g.ctypes.data, up.ctypes.data, x.size, tab.ctypes.data)
    pos = ((x.astype(np.float64) + 10.0) * 8191.0) * 0.05
    idx = np.clip(np.rint(pos), 0, 8190).astype(int)
    frac = pos - idx
    want = (tab[idx] + (tab[idx + 1] - tab[idx]) * frac) * 2.0
    np.testing.assert_allclose(g, want, rtol=1e-5, atol=1e-5)
    inside = (x > -10) & (x < 10)
    silu = x / (1 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(g[inside], 2 * silu[inside], atol=2 * 0.05)  # table error < 0.05


def test_libm_expf_restatement_in_library_matches_host_libm():
    import tie_amd
    if not os.path.exists(tie_amd.LIB_PATH):
        pytest.skip("libtie_hip.so not built")
    # every 13th binary32 in (-inf, 0] and [0, 89): softmax feeds x - max <= 0
    neg = np.arange(0x80000000, 0xff800001, 13, dtype=np.uint64).astype(np.uint32).view(np.float32)
    pos = np.arange(0, 0x42b20000, 13, dtype=np.uint32).view(np.float32)
    for part in (neg, pos):
        for c in range(0, part.size, 1 << 24):
            v = part[c:c + (1 << 24)]
            np.testing.assert_array_equal(bits(tie_amd.host_expf(v)), bits(bind.libm_expf(v)))
