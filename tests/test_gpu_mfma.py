"""GPU parity of the MFMA (grouped bf16 GEMM) path, called through the C ABI.

Routing (logits, top-k, gate weights) is computed in exact fp32 on both paths,
so selected experts and gate weights must equal the oracle bit for bit.  The
expert products run on bf16 matrix cores, so outputs are checked two ways:

  * against a float64 model of the same arithmetic (weights dequantised in
    fp32 as TIE does, rounded to bf16 -- Q4_K and Q6_K weights run on the
    f16 matrix cores instead, emulated exactly, with x in f16 and h as
    f16(h / 256) * 256; other activations rounded to bf16; TIE's table
    SwiGLU; y rounded to bf16) -- this pins the kernels' tiling, operand
    layouts (including the f16 path's K permutation) and epilogue: relative
    L2 error <= 2e-3;
  * against the fp32 oracle (TIE's own arithmetic) -- the bf16 rounding
    error, reported and bounded: relative L2 error <= 2e-2 for Q4_K/Q6_K
    weights, and max |err| <= 1e-3 for BF16 weights (activations split into
    two bf16 parts).
"""
import numpy as np
import pytest

import tie_amd
from conftest import bits, synth_layer
from oracle import bind
from tie_amd import synth

pytestmark = pytest.mark.gpu


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


def q4k_f16(buf):
    """Q4_K weights as the f16 gate/up kernels form them, divided by their
    factor 256: per sub-block D = d*sc and M = -dmin*m in fp32 (exact), times
    256 rounded to f16, then code*D16 + M16 rounded once to f16 (v_pk_fma_f16).
    Super-block layout (TIE's block_q4_K): d, dmin (f16), 12 scale bytes, 128
    code bytes; sub-block 2g holds the low and 2g+1 the high nibbles of code
    bytes 32g..32g+31."""
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
    D = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    M = -(dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
    D16 = f16(D * 256).astype(np.float64)
    M16 = f16(M * 256).astype(np.float64)
    qs = b[:, 16:].reshape(nb, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float64)
    W = (q * D16[:, :, None] + M16[:, :, None]).astype(np.float16)  # exact in float64, one rounding
    return W.astype(np.float32).reshape(-1) / 256


def q6k_f16(buf):
    """Q6_K weights as the f16 kernels form them, divided by their factor 256:
    D = d*sc in fp32 (exact), D*256 rounded to f16, then (code - 32)*D16
    rounded once to f16 (v_pk_mul_f16).  Super-block layout (TIE's
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
    D16 = f16((d[:, None] * s).astype(np.float32) * 256).astype(np.float64)
    W = ((q - 32).astype(np.float64) * D16).astype(np.float16)  # exact in float64, one rounding
    return W.astype(np.float32).reshape(-1) / 256


def quant_f16(buf, wtype):
    return q4k_f16(buf) if wtype == synth.Q4_K else q6k_f16(buf)


def dequant(buf, wtype, E, rows, inn):
    if wtype == synth.BF16:
        return synth.bf16_bits_to_f32(np.ascontiguousarray(buf).view(np.uint16)).reshape(E, rows, inn)
    out = np.empty(E * rows * inn, np.float32)
    fn = bind.oracle().orc_dequant_q4k if wtype == synth.Q4_K else bind.oracle().orc_dequant_q6k
    fn(np.ascontiguousarray(buf).ctypes.data, E * rows * inn, out.ctypes.data)
    return out.reshape(E, rows, inn)


def model(layer, x, k, idx, w, tab, split):
    """float64 model of the MFMA path given the (exact) routing."""
    d, F, E = layer.d, layer.F, layer.E
    Wg = dequant(layer.gate, layer.gate_type, E, F, d)
    Wu = dequant(layer.up, layer.up_type, E, F, d)
    Wd = dequant(layer.down, layer.down_type, E, d, F)
    xa = x
    quant = (synth.Q4_K, synth.Q6_K)
    h16 = layer.down_type in quant  # h as f16 * 2^-8 (down on f16 operands)
    if not split:
        if layer.gate_type in quant:
            # f16 operands
            Wg = quant_f16(layer.gate, layer.gate_type).reshape(E, F, d)
            Wu = quant_f16(layer.up, layer.up_type).reshape(E, F, d)
            xa = f16(x)
        else:
            Wg, Wu, xa = bf16(Wg), bf16(Wu), bf16(x)
    if h16:
        Wd = quant_f16(layer.down, layer.down_type).reshape(E, d, F)
    elif not split:
        Wd = bf16(Wd)
    out = np.zeros(x.shape, np.float64)
    for t in range(x.shape[0]):
        for j in range(k):
            e = idx[t, j]
            if e < 0:
                continue
            g = (Wg[e].astype(np.float64) @ xa[t].astype(np.float64)).astype(np.float32)
            u = (Wu[e].astype(np.float64) @ xa[t].astype(np.float64)).astype(np.float32)
            bind.oracle().orc_swiglu(g.ctypes.data, u.ctypes.data, F, tab.ctypes.data)
            h = f16(g / 256) * 256 if h16 else g if split else bf16(g)
            y = Wd[e].astype(np.float64) @ h.astype(np.float64)
            if not split:
                y = bf16(y.astype(np.float32)).astype(np.float64)  # stored as bf16 for the combine
            out[t] += float(w[t, j]) * y
    return out


def rel_l2(a, b):
    return float(np.linalg.norm((a - b).ravel()) / max(np.linalg.norm(np.asarray(b).ravel()), 1e-30))


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


@pytest.mark.parametrize("shape", [(256, 256, 16, 4, 40), (512, 512, 8, 2, 300), (2048, 768, 128, 8, 64)])
@pytest.mark.parametrize("types", [(synth.Q4_K, synth.Q6_K), (synth.Q6_K, synth.Q4_K)])
def test_quantised_against_bf16_model_and_oracle(shape, types):
    d, F, E, k, T = shape
    layer = synth_layer(31 + d + T, d, F, E, types[0], types[1], None)
    x = synth.make_input(31 + T, T, d)
    out, idx, w = run_mfma(layer, x, k)
    ro, ri, rw = bind.moe_block(layer, x, k)
    np.testing.assert_array_equal(idx, ri)
    np.testing.assert_array_equal(bits(w), bits(rw))
    tab = bind.silu_table()
    m = model(layer, x, k, ri, rw, tab, split=False)
    e_model = rel_l2(out, m)
    e_oracle = rel_l2(out, ro)
    print("rel L2 vs bf16 model %.3g, vs fp32 oracle %.3g; max|err|/max|ref| vs oracle %.3g" % (
        e_model, e_oracle, np.abs(out - ro).max() / np.abs(ro).max()), flush=True)
    assert e_model <= 2e-3
    assert e_oracle <= 2e-2


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
    np.testing.assert_array_equal(idx, ri)
    np.testing.assert_array_equal(bits(w), bits(rw))
    err = np.abs(out - ro).max()
    print("bf16 weights: max|err| %.3g (max|out| %.3g), rel L2 %.3g" % (err, np.abs(ro).max(), rel_l2(out, ro)),
          flush=True)
    assert err <= 1e-3


def test_full_prefill_30b_routing_exact_and_sampled_outputs():
    c = synth.CONFIGS["30b_t2048"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None)
    x = synth.make_input(c["seed"], c["T"], c["d"])
    out, idx, w = run_mfma(layer, x, c["k"])
    sample = np.arange(0, c["T"], 32)  # every 32nd token through the oracle
    ro, ri, rw = bind.moe_block(layer, x[sample], c["k"])
    np.testing.assert_array_equal(idx[sample], ri)
    np.testing.assert_array_equal(bits(w[sample]), bits(rw))
    e = rel_l2(out[sample], ro)
    print("T=2048 sampled rel L2 vs oracle %.3g" % e, flush=True)
    assert e <= 2e-2


def test_lfm2_prefill_routing_exact():
    """Sigmoid routing on the MFMA path (separate selection kernel at large
    T): selection and weights bit-exact against the oracle, outputs within
    the bf16 bound."""
    c = synth.CONFIGS["lfm2_t32"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None, 1, c["probs_bias"])
    T = 300
    x = synth.make_input(c["seed"] + 5, T, c["d"])
    out, idx, w = run_mfma(layer, x, c["k"])
    ro, ri, rw = bind.moe_block(layer, x, c["k"])
    np.testing.assert_array_equal(idx, ri)
    np.testing.assert_array_equal(bits(w), bits(rw))
    e = rel_l2(out, ro)
    print("lfm2 T=300 rel L2 vs oracle %.3g" % e, flush=True)
    assert e <= 2e-2
