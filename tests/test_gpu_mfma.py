"""GPU parity of the MFMA (grouped matrix-core GEMM) path, called through the
C ABI.

Routing (logits, top-k, gate weights) is computed in exact fp32 on both paths,
so selected experts and gate weights must equal the oracle bit for bit.  The
expert products run on the 16-bit matrix cores, so outputs are checked two
ways:

  * against a float64 model of the same arithmetic (the kernels' operands
    emulated exactly: Q4_K / Q6_K weights dequantised in packed f16 with
    their factor 256, x rounded to f16, h rounded to an 11-bit significand
    (f16 scaled by the layer's power of two), y likewise; BF16
    weights with activations split into two bf16 parts; TIE's table SwiGLU)
    -- this pins the kernels' tiling, operand layouts (including the K
    permutation), pipelines and epilogues;
  * against the fp32 oracle (TIE's own arithmetic): the 16-bit rounding
    error, bounded at about twice what it measures.

Tokens whose activations leave the f16 range are recomputed in TIE's exact
arithmetic; their rows must equal the oracle bit for bit.
"""
import numpy as np
import pytest

import tie_amd
from conftest import bits, synth_layer
from oracle import bind
from tie_amd import synth

pytestmark = pytest.mark.gpu

# Quantised weights against the fp32 oracle: relative L2 and max |err| /
# max |ref| both <= 1e-3 (the f16 operands' rounding: about 5.5e-4 of
# either, from the weights, x, h and y), and rel. L2 against the float64
# model of the kernels' own operands
ORACLE_RL2 = 1e-3
ORACLE_MAXREL = 1e-3
MODEL_RL2 = 3e-4
# BF16 weights (activations split into two bf16 parts): the north star's max
# |err| bound (values O(1)), and rel. L2 (measured 4.4e-6 .. 4.6e-6)
BF16_MAXABS = 1e-3
BF16_RL2 = 2e-5


@pytest.fixture(scope="module", autouse=True)
def device():
    import torch
    assert torch.cuda.is_available(), "GPU test without a GPU"
    tie_amd.init(0)
    yield
    tie_amd.shutdown()


def bf16(a):
    return synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(np.asarray(a, np.float32)))


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def sig11(a):
    """Round to an 11-bit significand (f16's), exponent unbounded: f16 of a
    value scaled into f16's normal range by a power of two, scaled back."""
    a = np.asarray(a, np.float64)
    m, e = np.frexp(a)
    return np.ldexp(np.round(m * 2048.0) / 2048.0, e)


def q4k_f16(buf, fold=False):
    """Q4_K weights as the f16 kernels form them, divided by their factor
    256: per sub-block M = -dmin*m*256 rounded to f16, then (code*sc)*(d*256)
    + M16 rounded once to f16 (code*sc and d*256 exact in f16;
    v_pk_fma_f16); with fold (the 32-row gate/up tile kernels: MFMAs on
    code*sc, d*256 applied per block in fp32, M16 times the activations'
    sub-block sums) not rounded.
    Super-block layout (TIE's block_q4_K): d, dmin (f16), 12 scale bytes,
    128 code bytes; sub-block 2g holds the low and 2g+1 the high nibbles of
    code bytes 32g..32g+31."""
    b = np.frombuffer(np.ascontiguousarray(buf).tobytes(), np.uint8).reshape(-1, 144)
    nb = b.shape[0]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.int32)
    sc = np.empty((nb, 8), np.int32)
    mn = np.empty((nb, 8), np.int32)
    for j in range(4):
        sc[:, j] = s[:, j] & 63
        mn[:, j] = s[:, j + 4] & 63
    for j in range(4, 8):
        sc[:, j] = (s[:, j + 4] & 15) | ((s[:, j - 4] >> 6) << 4)
        mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    D16 = (d[:, None].astype(np.float64) * 256) * sc.astype(np.float64)  # exact: (code sc) (d 256) in the fma
    M = -(dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
    M16 = f16(M * 256).astype(np.float64)
    qs = b[:, 16:].reshape(nb, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float64)
    W = q * D16[:, :, None] + M16[:, :, None]  # exact in float64
    if not fold:
        W = W.astype(np.float16).astype(np.float32)  # one rounding
    return W.reshape(-1) / 256


def q6k_f16(buf, dfold=False):
    """Q6_K weights as the f16 kernels form them, divided by their factor 256:
    (code - 32)*sc in f16 (exact for |sc| <= 64, as in these blocks), times
    d*256 (exact), rounded once to f16 (v_pk_mul_f16); with dfold (the 32-row
    tile kernels, which apply d*256 per 256-K block to an fp32 block sum) not
    rounded.  Super-block layout (TIE's
    block_q6_K): ql[128], qh[64], int8 scales[16], d (f16); half n, l < 32:
    weights 128n + l + 32i take ql nibble (ql[64n + l + 32(i%2)], low for
    i < 2), qh bits 2i of qh[32n + l], scale 8n + l//16 + 2i."""
    b = np.frombuffer(np.ascontiguousarray(buf).tobytes(), np.uint8).reshape(-1, 210)
    nb = b.shape[0]
    ql, qh = b[:, 0:128].astype(np.int32), b[:, 128:192].astype(np.int32)
    sc = b[:, 192:208].copy().view(np.int8).astype(np.float32)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    q = np.empty((nb, 256), np.int32)
    s = np.empty((nb, 256), np.float32)
    l = np.arange(32)
    for n in range(2):
        for i in range(4):
            nib = ql[:, 64 * n + l + 32 * (i % 2)]
            nib = nib & 15 if i < 2 else nib >> 4
            q[:, 128 * n + 32 * i + l] = nib | (((qh[:, 32 * n + l] >> (2 * i)) & 3) << 4)
            s[:, 128 * n + 32 * i + l] = sc[:, 8 * n + l // 16 + 2 * i]
    qs = f16((q - 32).astype(np.float32) * s).astype(np.float64)  # (code - 32) sc: exact when |sc| <= 64
    W = qs * (d[:, None].astype(np.float64) * 256)
    if not dfold:
        W = W.astype(np.float16).astype(np.float32)  # one rounding
    return W.reshape(-1) / 256


QUANT = (synth.Q4_K, synth.Q6_K)
TINY_AVG = 16  # pairs per expert on average up to which the kernels take 32-row tiles


def expert_weights(buf, wtype, e, rows, inn, f16_ops, dfold=False, qfold=False):
    """Expert e's [rows][inn] weights as the kernels' operands (dfold: the
    32-row tile kernels' Q6_K form, q6k_f16; qfold: their Q4_K gate/up form,
    q4k_f16)."""
    nbytes = rows * synth.row_bytes(wtype, inn)
    raw = np.ascontiguousarray(np.frombuffer(np.ascontiguousarray(buf).tobytes(), np.uint8,
                                             count=nbytes, offset=e * nbytes))
    if wtype == synth.BF16:
        return synth.bf16_bits_to_f32(raw.view(np.uint16)).reshape(rows, inn)
    if f16_ops:
        return (q4k_f16(raw, qfold) if wtype == synth.Q4_K else q6k_f16(raw, dfold)).reshape(rows, inn)
    out = np.empty(rows * inn, np.float32)
    fn = bind.oracle().orc_dequant_q4k if wtype == synth.Q4_K else bind.oracle().orc_dequant_q6k
    fn(raw.ctypes.data, rows * inn, out.ctypes.data)
    return bf16(out).reshape(rows, inn)


def model(layer, x, idx, w, tab):
    """float64 model of the MFMA path given the (exact) routing, grouped by
    expert (matrix products per expert)."""
    d, F = layer.d, layer.F
    split = layer.gate_type == synth.BF16       # activations as bf16 hi + lo (exact to ~16 bits)
    h16 = layer.down_type in QUANT               # h in f16 (scaled) for the f16 down kernels
    if split:
        xa = x.astype(np.float64)
    elif layer.gate_type in QUANT:
        xa = f16(x).astype(np.float64)
    else:
        xa = bf16(x).astype(np.float64)
    out = np.zeros(x.shape, np.float64)
    # 32-row tiles (at most TINY_AVG pairs per expert on average) for both
    # quantised kernels
    tiny = idx.size <= TINY_AVG * layer.E
    for e in np.unique(idx[idx >= 0]):
        t, j = np.nonzero(idx == e)
        Wg = expert_weights(layer.gate, layer.gate_type, e, F, d, True, tiny, tiny)
        Wu = expert_weights(layer.up, layer.up_type, e, F, d, True, tiny, tiny)
        Wd = expert_weights(layer.down, layer.down_type, e, d, F, h16, tiny)
        X = xa[t]
        g = np.ascontiguousarray((X @ Wg.T.astype(np.float64)).astype(np.float32))
        u = np.ascontiguousarray((X @ Wu.T.astype(np.float64)).astype(np.float32))
        bind.oracle().orc_swiglu(g.ctypes.data, u.ctypes.data, g.size, tab.ctypes.data)
        if h16:
            h = sig11(g)
        elif split:
            h = g.astype(np.float64)
        else:
            h = bf16(g).astype(np.float64)
        y = h @ Wd.T.astype(np.float64)
        # stored for the combine as f16 scaled by the layer's power of two
        # (an 11-bit significand), fp32 with BF16 weights
        y = sig11(y.astype(np.float32)) if h16 else y.astype(np.float32).astype(np.float64)
        np.add.at(out, t, w[t, j].astype(np.float64)[:, None] * y)
    return out


def rel_l2(a, b):
    return float(np.linalg.norm((np.asarray(a, np.float64) - b).ravel()) /
                 max(np.linalg.norm(np.asarray(b, np.float64).ravel()), 1e-30))


def report(tag, out, ro):
    e = rel_l2(out, ro)
    mx = float(np.abs(out - ro).max())
    print("PARITY %s rel_l2=%.3e max_abs=%.3e max_ref=%.3e" % (tag, e, mx, float(np.abs(ro).max())), flush=True)
    return e, mx


def check_oracle(tag, out, ro):
    """The 16-bit operand bound against the fp32 oracle: rel. L2 and
    max |err| / max |ref| <= 1e-3."""
    e, mx = report(tag, out, ro)
    assert e <= ORACLE_RL2, (tag, e)
    assert mx <= ORACLE_MAXREL * float(np.abs(ro).max()), (tag, mx)
    return e, mx


def run_mfma(layer, x, k):
    import torch
    L = tie_amd.Layer.from_synth(layer)
    xd = torch.from_numpy(x).cuda()
    T = x.shape[0]
    out = torch.empty_like(xd)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    print("mfma case d=%d F=%d E=%d T=%d k=%d types=%d/%d" % (layer.d, layer.F, layer.E, T, k, layer.gate_type,
                                                                layer.down_type), flush=True)
    L.forward(xd, T, k, out, idx, w, flags=tie_amd.PATH_MFMA)
    torch.cuda.synchronize()
    res = out.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()
    L.close()
    return res


def check_routing(idx, w, ri, rw):
    np.testing.assert_array_equal(idx, ri)
    np.testing.assert_array_equal(bits(w), bits(rw))


# (d, F, E, k, T): small shapes, the 30B shape at few pairs per expert
# (T = 32 and 7: one work item per expert and column slab, h by expert;
# T = 64: the scanned tile list), 25 pairs per expert (64-row gate/up
# tiles), and few experts at T = 1024 (256 pairs per expert: full 160-row
# gate/up tiles, the cross-stage software pipeline, several tiles per expert)
@pytest.mark.parametrize("shape", [(256, 256, 16, 4, 40), (256, 256, 16, 4, 100), (512, 512, 8, 2, 300),
                                   (2048, 768, 128, 8, 64),
                                   (2048, 768, 128, 8, 32), (512, 512, 16, 4, 7), (2048, 768, 8, 2, 1024)])
@pytest.mark.parametrize("types", [(synth.Q4_K, synth.Q6_K), (synth.Q6_K, synth.Q4_K)])
def test_quantised_against_model_and_oracle(shape, types):
    d, F, E, k, T = shape
    layer = synth_layer(31 + d + T, d, F, E, types[0], types[1], None)
    x = synth.make_input(31 + T, T, d)
    out, idx, w = run_mfma(layer, x, k)
    ro, ri, rw = bind.moe_block(layer, x, k)
    check_routing(idx, w, ri, rw)
    m = model(layer, x, ri, rw, bind.silu_table())
    e_model = rel_l2(out, m)
    print("rel L2 vs kernel model %.3e" % e_model, flush=True)
    assert e_model <= MODEL_RL2
    check_oracle("q_%d_%d_%d_%d_%d_%d" % (d, F, E, k, T, types[0]), out, ro)


@pytest.mark.parametrize("case", ["full_tiles", "one_token", "wide_E"])
def test_direct_items_edges(case):
    """Batches of up to 32 tokens (one work item per expert and column slab,
    h by expert) at their edges: 32 nearly equal tokens (the same experts
    for all: full 32-row tiles), one token on the matrix cores, and 1024
    experts (a grid of 1032 item rows, most experts without pairs)."""
    if case == "full_tiles":
        d, F, E, k, T = 2048, 768, 128, 8, 32
        rng = np.random.default_rng(95)
        base = synth.make_input(96, 1, d)
        x = (base * (1 + 1e-4 * rng.standard_normal((T, d)))).astype(np.float32)
    elif case == "one_token":
        d, F, E, k, T = 2048, 768, 128, 8, 1
        x = synth.make_input(97, T, d)
    else:
        d, F, E, k, T = 256, 256, 1024, 8, 16
        x = synth.make_input(98, T, d)
    layer = synth_layer(99 + E + T, d, F, E, synth.Q4_K, synth.Q6_K, None)
    out, idx, w = run_mfma(layer, x, k)
    ro, ri, rw = bind.moe_block(layer, x, k)
    check_routing(idx, w, ri, rw)
    if case == "full_tiles":
        # the same experts for every token (most of them): full tiles
        assert max(int((ri == e).sum()) for e in np.unique(ri)) == T
    m = model(layer, x, ri, rw, bind.silu_table())
    e_model = rel_l2(out, m)
    print("rel L2 vs kernel model %.3e" % e_model, flush=True)
    assert e_model <= MODEL_RL2
    check_oracle("direct_%s" % case, out, ro)


@pytest.mark.parametrize("T,zipf", [(48, None), (200, 1.2)])
def test_bf16_weights_split_activations(T, zipf):
    d, F, E, k = 512, 256, 16, 4
    layer = synth_layer(77 + T, d, F, E, synth.BF16, synth.BF16, zipf)
    x = synth.make_input(77, T, d)
    import torch
    L = tie_amd.Layer.from_synth(layer)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    L.forward(xd, T, k, out, idx, w, flags=tie_amd.PATH_MFMA)
    torch.cuda.synchronize()
    out, idx, w = out.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()
    L.close()
    ro, ri, rw = bind.moe_block(layer, x, k)
    check_routing(idx, w, ri, rw)
    e, err = report("bf16_T%d" % T, out, ro)
    assert err <= BF16_MAXABS and e <= BF16_RL2


@pytest.mark.parametrize("cfg", ["30b_t2048", "235b_t1024"])
@pytest.mark.parametrize("scaled", [False, True])
def test_full_prefill_all_tokens(cfg, scaled):
    """The headline prefill shapes at full size: every token's selection
    bit-exact, every output row within the 16-bit bound.  scaled: the
    weights' fp16 super-block scales times 2^-6 (gate/up) and 2^-8 (down),
    which brings the block's outputs from O(1e6) to O(1) (RMS about 0.5,
    weights near a real model's ~N(0, 0.02)) and |g| near SiLU's curved
    range; the relative bounds hold there too."""
    c = synth.CONFIGS[cfg]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None)
    if scaled:
        import copy
        base, layer = layer, copy.copy(layer)
        layer.gate = scaled_scales(base.gate, base.gate_type, 2.0 ** -6)
        layer.up = scaled_scales(base.up, base.up_type, 2.0 ** -6)
        layer.down = scaled_scales(base.down, base.down_type, 2.0 ** -8)
    x = synth.make_input(c["seed"], c["T"], c["d"])
    out, idx, w = run_mfma(layer, x, c["k"])
    ro, ri, rw = bind.moe_block(layer, x, c["k"])
    check_routing(idx, w, ri, rw)
    assert np.isfinite(out).all()
    check_oracle(cfg + ("_o1" if scaled else ""), out, ro)


def test_full_bf16_zipf_t512():
    """30B shape, BF16 experts, Zipf-biased routing, T = 512 on the matrix
    cores (the split-activation kernels at d = 2048, E = 128 with imbalanced
    tiles): selection bit-exact, max |err| <= 1e-3."""
    c = synth.CONFIGS["30b_bf16_zipf_t512"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], c["zipf"])
    x = synth.make_input(c["seed"], c["T"], c["d"])
    out, idx, w = run_mfma(layer, x, c["k"])
    ro, ri, rw = bind.moe_block(layer, x, c["k"])
    check_routing(idx, w, ri, rw)
    counts = np.bincount(ri.ravel(), minlength=c["E"])
    print("zipf: busiest expert %d pairs, %d experts idle" % (counts.max(), int((counts == 0).sum())), flush=True)
    e, err = report("30b_bf16_zipf_t512", out, ro)
    assert err <= BF16_MAXABS and e <= BF16_RL2


def scaled_scales(buf, wtype, factor):
    """A copy of a Q4_K / Q6_K tensor with every fp16 super-block scale
    (Q4_K d and dmin, Q6_K d) multiplied by factor (a power of two)."""
    size = 144 if wtype == synth.Q4_K else 210
    b = np.frombuffer(np.ascontiguousarray(buf).tobytes(), np.uint8).reshape(-1, size).copy()
    cols = [(0, 2), (2, 4)] if wtype == synth.Q4_K else [(208, 210)]
    for a, z in cols:
        v = b[:, a:z].copy().view(np.float16).astype(np.float32) * np.float32(factor)
        b[:, a:z] = v.astype(np.float16).view(np.uint8)
    return b.reshape(-1)


def test_small_activations():
    """Weights 64x smaller than the synthetic default (closer to real
    models): |h| ~ 1e-3.  The layer's h scale keeps those values normal f16
    numbers, so the error against the oracle stays at the 16-bit level."""
    import copy
    base = synth_layer(91, 2048, 768, 16, synth.Q4_K, synth.Q6_K, None)
    layer = copy.copy(base)
    layer.gate = scaled_scales(base.gate, synth.Q4_K, 1.0 / 64)
    layer.up = scaled_scales(base.up, synth.Q4_K, 1.0 / 64)
    x = synth.make_input(91, 256, 2048)
    out, idx, w = run_mfma(layer, x, 4)
    ro, ri, rw = bind.moe_block(layer, x, 4)
    check_routing(idx, w, ri, rw)
    check_oracle("small_h", out, ro)


@pytest.mark.parametrize("seed,E,T,far", [(93, 16, 160, None), (94, 32, 300, 297)])
def test_out_of_range_tokens_recomputed_exactly(seed, E, T, far):
    """Tokens whose x (|x| >= 65504, NaN) or scaled h leave the f16 range
    are recomputed in TIE's exact arithmetic: their rows equal the oracle
    bit for bit, and no other row changes.  E = 16, T = 160: the
    routing kernel converts x and flags the tokens; E = 32, T = 300: the
    tiled logits kernel does (T > 256), with a flagged token in the last,
    partial 16-token tile."""
    layer = synth_layer(seed, 512, 512, E, synth.Q4_K, synth.Q6_K, None)
    k = 4
    x = synth.make_input(seed, T, 512)
    base_out, _, _ = run_mfma(layer, x, k)
    x2 = x.copy()
    x2[5] *= np.float32(1e5)     # x beyond f16
    x2[9] *= np.float32(200.0)   # x fits f16, h ~ 4e4 x typical: beyond
    x2[17, 3] = np.nan           # NaN logits: no expert, output 0
    bad = [5, 9, 17]
    if far is not None:
        x2[far, 200] = np.float32(7e4)  # one value beyond f16 in a late K chunk
        bad.append(far)
    out, idx, w = run_mfma(layer, x2, k)
    ro, ri, rw = bind.moe_block(layer, x2, k)
    check_routing(idx, w, ri, rw)
    for t in bad:
        np.testing.assert_array_equal(bits(out[t]), bits(ro[t]), err_msg="row %d" % t)
    assert (out[17] == 0).all()
    rest = np.setdiff1d(np.arange(T), bad)
    np.testing.assert_array_equal(bits(out[rest]), bits(base_out[rest]))
    assert np.isfinite(out[rest]).all()


def test_lfm2_prefill_routing_exact():
    """Sigmoid routing on the MFMA path (separate selection kernel at large
    T): selection and weights bit-exact against the oracle, outputs within
    the 16-bit bound."""
    c = synth.CONFIGS["lfm2_t32"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None, 1, c["probs_bias"])
    T = 300
    x = synth.make_input(c["seed"] + 5, T, c["d"])
    out, idx, w = run_mfma(layer, x, c["k"])
    ro, ri, rw = bind.moe_block(layer, x, c["k"])
    check_routing(idx, w, ri, rw)
    check_oracle("lfm2_T300", out, ro)


def test_out_of_range_residual_in_place():
    """The FFN half (RMSNorm, block, residual) on the MFMA path with every
    token's normed x beyond the f16 range (one huge ffn_norm weight): every
    row is recomputed exactly, also when the residual add updates the
    hidden state in place (the recomputation reads the hidden state as it
    was, so the combine must leave those rows alone): bit-exact against the
    oracle, in place and out of place."""
    import torch
    layer = synth_layer(95, 512, 512, 16, synth.Q4_K, synth.Q6_K, None)
    T, k = 100, 4
    hidden = synth.make_input(95, T, 512)
    norm = synth.make_norm_weight(95, 512)
    norm[7] = np.float32(1e6)
    rh, ri, rw = bind.qwen3_ffn(layer, hidden, k, norm, 1e-6)
    L = tie_amd.Layer.from_synth(layer)
    nd = torch.from_numpy(norm).cuda()
    for in_place in (False, True):
        hd = torch.from_numpy(hidden).cuda()
        out = hd if in_place else torch.empty_like(hd)
        idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w = torch.empty((T, k), dtype=torch.float32, device="cuda")
        L.forward_residual(hd, nd, 1e-6, T, k, None if in_place else out, idx, w, flags=tie_amd.PATH_MFMA)
        torch.cuda.synchronize()
        print("in place %s" % in_place, flush=True)
        check_routing(idx.cpu().numpy(), w.cpu().numpy(), ri, rw)
        np.testing.assert_array_equal(bits(out.cpu().numpy()), bits(rh), err_msg="in place %s" % in_place)
    L.close()


@pytest.mark.parametrize("wtype", QUANT)
def test_dense_mat_mat_mfma(wtype):
    """tie_hip_mat_mat on the matrix cores (TIE_HIP_PATH_MFMA; the default
    keeps the exact row kernels): against the float64 model of its
    operands (x in f16, the f16 weights of q4k_f16 / q6k_f16) and against
    TIE's row kernels (the fp32 oracle); a token whose x leaves the f16 range
    is computed exactly instead (bit-exact).  The small matrix makes the
    launcher shrink the tiles (32 to 128 rows: every token count here runs
    tiles of fewer rows than the kernel's maximum, with ragged last tiles)."""
    import torch
    rows, in_dim = 512, 1024
    rng = np.random.default_rng(60 + wtype)
    w = synth.expert_tensor(rng, wtype, 1, rows, in_dim)
    W16 = expert_weights(w, wtype, 0, rows, in_dim, True).astype(np.float64)
    M = tie_amd.Matrix(w, wtype, rows, in_dim)
    for T, flags in ((65, tie_amd.PATH_MFMA), (200, tie_amd.PATH_MFMA), (7, tie_amd.PATH_MFMA),
                     (32, tie_amd.PATH_MFMA), (130, tie_amd.PATH_MFMA)):
        x = synth.make_input(61 + T, T, in_dim)
        x[3] *= np.float32(1e5)  # beyond f16: recomputed exactly
        print("dense mfma type=%d T=%d" % (wtype, T), flush=True)
        xd = torch.from_numpy(x).cuda()
        out = torch.empty((T, rows), device="cuda")
        M.mat_mat(xd, T, out, flags=flags)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ro = bind.mat_mat(x, w, wtype, rows)
        np.testing.assert_array_equal(bits(got[3]), bits(ro[3]), err_msg="flagged row")
        rest = np.setdiff1d(np.arange(T), [3])
        ref = f16(x[rest]).astype(np.float64) @ W16.T
        e_model = rel_l2(got[rest], ref)
        assert e_model <= MODEL_RL2, e_model
        check_oracle("dense_mfma t%d T=%d" % (wtype, T), got[rest], ro[rest])
    # the default (TIE_HIP_PATH_AUTO) keeps TIE's row kernels at any T: bit-exact
    x = synth.make_input(70, 130, in_dim)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((130, rows), device="cuda")
    M.mat_mat(xd, 130, out, flags=tie_amd.PATH_AUTO)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out.cpu().numpy()), bits(bind.mat_mat(x, w, wtype, rows)))
    M.close()


def test_dense_mat_mat_mfma_limits():
    """The matrix-core dense path is refused for what it cannot run (F32,
    rows not a multiple of 256) when asked for, and not taken by default:
    the default then runs TIE's row kernels (bit-exact)."""
    import torch
    rows, in_dim, T = 320, 512, 100
    rng = np.random.default_rng(66)
    w = synth.expert_tensor(rng, synth.Q4_K, 1, rows, in_dim)
    M = tie_amd.Matrix(w, synth.Q4_K, rows, in_dim)
    x = synth.make_input(66, T, in_dim)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((T, rows), device="cuda")
    with pytest.raises(tie_amd.TieError):
        M.mat_mat(xd, T, out, flags=tie_amd.PATH_MFMA)
    M.mat_mat(xd, T, out, flags=tie_amd.PATH_AUTO)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out.cpu().numpy()), bits(bind.mat_mat(x, w, synth.Q4_K, rows)))
    M.close()


def test_f16_scales_from_device_and_host_sources():
    """The powers of two the matrix-core path scales h and y by are chosen
    at upload from samples of the gate and down weights; a layer uploaded
    from device memory gets the same ones as from host memory, and they
    put the typical |h|, |y| well inside f16's range (30B shape: h near
    2^14 before scaling, y near 2^21)."""
    import torch
    c = synth.CONFIGS["30b_t2048"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None)
    Lh = tie_amd.Layer.from_synth(layer)
    dev = [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (layer.router, layer.gate, layer.up, layer.down)]
    Ld = tie_amd.Layer(layer.d, layer.F, layer.E, *dev, layer.gate_type, layer.up_type, layer.down_type,
                       on_device=True)
    hs, ys = Lh.shifts()
    print("shifts host %s device %s" % ((hs, ys), Ld.shifts()), flush=True)
    assert Ld.shifts() == (hs, ys)
    assert 8 <= hs <= 16 and 12 <= ys <= 22
    Lh.close()
    Ld.close()


def test_auto_path_threshold():
    """TIE_HIP_PATH_AUTO: TIE's exact kernels up to tie_hip_exact_max_tokens()
    tokens (14 by default; bit-exact), the matrix cores above (the 16-bit
    bound), through the host drop-in."""
    assert tie_amd.lib().tie_hip_exact_max_tokens() == 14
    c = synth.CONFIGS["30b_t32"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None)
    for T in (14, 15, 32):
        x = synth.make_input(400 + T, T, c["d"])
        print("auto T=%d" % T, flush=True)
        out, idx, w = tie_amd.moe_ffn(x, layer, c["k"])
        ro, ri, rw = bind.moe_block(layer, x, c["k"])
        check_routing(idx, w, ri, rw)
        if T <= 14:
            np.testing.assert_array_equal(bits(out), bits(ro))
        else:
            check_oracle("auto_T%d" % T, out, ro)


def test_graph_replays_of_batches():
    """Batched forwards captured in one HIP graph -- the matrix-core path at
    T = 32 (one work item per expert and slab) and at T = 300 (tiled router
    logits, selection bytes and bucket_plan, one token beyond the f16 range
    recomputed exactly), and the exact path at T = 8 -- replayed four times
    with eager work on the library stream in between: every replay equals
    the eager result bit for bit (no step relies on memory cleared outside
    its own kernels)."""
    import torch
    cases = [(synth_layer(90, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None), 32, 8, tie_amd.PATH_MFMA),
             (synth_layer(91, 512, 512, 32, synth.Q4_K, synth.Q6_K, None), 300, 4, tie_amd.PATH_MFMA),
             (synth_layer(92, 512, 256, 16, synth.Q6_K, synth.Q4_K, None), 8, 4, tie_amd.PATH_EXACT)]
    Ls = [tie_amd.Layer.from_synth(c[0]) for c in cases]
    xs = []
    for i, (layer, T, k, _) in enumerate(cases):
        x = synth.make_input(93 + i, T, layer.d)
        if T == 300:
            x[7] *= np.float32(1e5)
        xs.append(torch.from_numpy(x).cuda())
    outs = [torch.empty_like(x) for x in xs]
    idxs = [torch.empty((c[1], c[2]), dtype=torch.int32, device="cuda") for c in cases]
    s = torch.cuda.Stream()

    def run_all():
        for L, x, o, ix, (layer, T, k, fl) in zip(Ls, xs, outs, idxs, cases):
            L.forward(x, T, k, o, ix, None, flags=fl, stream=s.cuda_stream)

    with torch.cuda.stream(s):
        run_all()
    torch.cuda.synchronize()
    eager = [o.cpu().numpy() for o in outs]
    eager_idx = [ix.cpu().numpy() for ix in idxs]
    for i, (layer, T, k, fl) in enumerate(cases):
        ro, ri, _ = bind.moe_block(layer, xs[i].cpu().numpy(), k)
        np.testing.assert_array_equal(eager_idx[i], ri)
        if fl == tie_amd.PATH_EXACT:
            np.testing.assert_array_equal(bits(eager[i]), bits(ro))
        else:
            check_oracle("graph_eager_%d" % i, eager[i], ro)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        run_all()
    for rep in range(4):
        for o, ix in zip(outs, idxs):
            o.fill_(-1.0)
            ix.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print("graph replay %d" % rep, flush=True)
        for i in range(len(cases)):
            np.testing.assert_array_equal(bits(outs[i].cpu().numpy()), bits(eager[i]),
                                          err_msg="replay %d case %d" % (rep, i))
            np.testing.assert_array_equal(idxs[i].cpu().numpy(), eager_idx[i])
        # eager forwards between replays, on the library stream
        layer, T, k, _ = cases[rep % 3]
        tie_amd.moe_ffn(xs[rep % 3].cpu().numpy(), layer, k)
    del g
    for L in Ls:
        L.close()
