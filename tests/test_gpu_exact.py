"""GPU parity of the exact path: the HIP block, called through the C ABI,
against the CPU oracle on the same inputs -- bit for bit.

The oracle runs on this host's CPU and builds TIE's SiLU table with this
host's reciprocal instruction, which is also what the library uploads at
tie_hip_init(); the committed golden vectors pin the oracle itself (see
test_oracle.py) and are compared directly where the host CPU matches the one
they were made on.
"""
import numpy as np
import pytest

import tie_amd
from conftest import bits, golden_layer, host_cpu_identity, load_golden, synth_layer
from oracle import bind
from tie_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    import torch
    assert torch.cuda.is_available(), "GPU test without a GPU"
    tie_amd.init(0)
    # the host drop-in (TIE_HIP_PATH_AUTO) on the exact path for every batch
    # these tests run (up to 64 tokens)
    old = tie_amd.lib().tie_hip_exact_max_tokens()
    tie_amd.lib().tie_hip_set_exact_max_tokens(64)
    yield
    tie_amd.lib().tie_hip_set_exact_max_tokens(old)
    tie_amd.shutdown()


def golden_host_check(g):
    """Whether this host can compare against the golden outputs directly (its
    CPU builds the same SiLU / RSQRTSS tables as the one that made them);
    printed either way, so the log says which comparison ran."""
    here, made = host_cpu_identity(), str(g["cpu"])
    same = here == made
    print("golden outputs %s (host %s, vectors from %s)" % ("compared" if same else "skipped: other CPU", here, made),
          flush=True)
    return same


def assert_same(got, want, what):
    g, w = np.ascontiguousarray(got), np.ascontiguousarray(want)
    if g.dtype == np.float32:
        nz = bits(g) != bits(w)
        if nz.any():
            i = np.argwhere(nz)[0]
            raise AssertionError("%s: %d of %d differ, first at %s: got %r want %r (max abs diff %g)" % (
                what, int(nz.sum()), nz.size, tuple(i), g[tuple(i)], w[tuple(i)], float(np.max(np.abs(g - w)))))
    else:
        np.testing.assert_array_equal(g, w, err_msg=what)


def run_both(layer, x, k):
    print("case d=%d F=%d E=%d T=%d k=%d types=%d/%d" % (layer.d, layer.F, layer.E, x.shape[0], k,
                                                         layer.gate_type, layer.down_type), flush=True)
    out, idx, w = tie_amd.moe_ffn(x, layer, k)
    ro, ri, rw = bind.moe_block(layer, x, k)
    assert_same(idx, ri, "topk_idx")
    assert_same(w, rw, "topk_w")
    assert_same(out, ro, "out")
    return out, idx, w


def test_library_table_is_oracle_table():
    assert_same(tie_amd.silu_table_host(), bind.silu_table(), "silu table")


@pytest.mark.parametrize("name", ["gtiny_q4k_t8", "gtiny_q6k_q4k_t8", "gtiny_ties_t6", "g30b_q4k_t4",
                                  "g235b_e16_t2"])
def test_golden_cases(name):
    g = load_golden(name)
    layer = golden_layer(g)
    out, idx, w = run_both(layer, g["x"], int(g["k"]))
    assert_same(idx, g["topk_idx"], "golden topk_idx")
    assert_same(w, g["topk_w"], "golden topk_w")
    if golden_host_check(g):
        assert_same(out, g["out"], "golden out")


@pytest.mark.parametrize("name", ["glfm2_t4", "glfm2_sat_t6"])
def test_lfm2_golden_cases(name):
    """Sigmoid routing (tie_hip_moe_ffn_lfm2): bit-exact against the oracle
    (both use the scalar expf and IEEE division); against the compiled
    reference's vectors within the LFM2 bar (its sigmoid loop is vectorised
    under -ffast-math): selection equal, weights within 1e-6 relative."""
    g = load_golden(name)
    layer = golden_layer(g)
    out, idx, w = run_both(layer, g["x"], int(g["k"]))
    assert_same(idx, g["topk_idx"], "golden topk_idx")
    np.testing.assert_allclose(w, g["topk_w"], rtol=1e-6, atol=0)
    if golden_host_check(g):
        assert np.abs(out - g["out"]).max() <= 1e-6 * np.abs(g["out"]).max()


def test_lfm2_one_token_without_bias():
    """One token routes inside the gate/up workgroups (sigmoid mode, no
    selection bias), and E > 128 goes through the grouping kernel."""
    for E in (32, 200):
        layer = synth_layer(27 + E, 512, 256, E, synth.Q4_K, synth.Q6_K, None, 1, None)
        for T, k in [(1, 4), (1, 8), (7, 4)]:
            run_both(layer, synth.make_input(27 + T, T, 512), k)


@pytest.mark.parametrize("wtype", [synth.Q4_K, synth.Q6_K, synth.BF16, synth.F32])
def test_dense_mat_mat(wtype):
    """tie_hip_mat_mat (dispatch_mat_mat with F32 input) against the oracle's
    row kernels, bit for bit, for ragged token counts (T <= 4 on the
    row-block kernel, more on the grouped GEMV kernels)."""
    import torch
    rows, in_dim = 512, 1024
    rng = np.random.default_rng(40 + wtype)
    if wtype == synth.F32:
        w = rng.normal(0, 0.02, size=rows * in_dim).astype(np.float32)
    else:
        w = synth.expert_tensor(rng, wtype, 1, rows, in_dim)
    M = tie_amd.Matrix(w, wtype, rows, in_dim)
    for T in (1, 3, 4, 5, 37, 200):
        x = synth.make_input(41 + T, T, in_dim)
        print("dense case type=%d T=%d" % (wtype, T), flush=True)
        xd = torch.from_numpy(x).cuda()
        out = torch.empty((T, rows), device="cuda")
        M.mat_mat(xd, T, out, flags=tie_amd.PATH_EXACT)
        torch.cuda.synchronize()
        assert_same(out.cpu().numpy(), bind.mat_mat(x, w, wtype, rows), "dense out")
    M.close()


@pytest.mark.parametrize("wtype,rows,in_dim", [(synth.Q6_K, 33024, 2048), (synth.Q4_K, 33024, 2048),
                                               (synth.Q6_K, 41024, 1536), (synth.Q4_K, 16448, 4096),
                                               (synth.Q4_K, 4096, 16384)])
def test_dense_stream(wtype, rows, in_dim):
    """One token through a tall matrix (the LM head's shape class): at
    rows x blocks / 64 >= 4096 units tie_hip_mat_mat streams units of 64 /
    nb rows through persistent waves (dense_stream_kernel), including block
    counts that do not divide 64 (nb = 6: ten rows per unit, four lanes
    idle), the largest input (nb = 64: one row per unit, the row sum by
    lane shuffles) and a last unit past the matrix's end; bit for bit with
    the oracle."""
    import torch
    rng = np.random.default_rng(50 + wtype + in_dim)
    w = synth.expert_tensor(rng, wtype, 1, rows, in_dim)
    M = tie_amd.Matrix(w, wtype, rows, in_dim)
    x = synth.make_input(51 + in_dim, 1, in_dim)
    x[0, 5] = -0.0
    print("dense stream case type=%d rows=%d in=%d" % (wtype, rows, in_dim), flush=True)
    xd = torch.from_numpy(x).cuda()
    out = torch.full((1, rows), float("nan"), device="cuda")
    for _ in range(2):
        M.mat_mat(xd, 1, out)
    torch.cuda.synchronize()
    assert_same(out.cpu().numpy(), bind.mat_mat(x, w, wtype, rows), "dense stream out")
    M.close()


@pytest.mark.parametrize("name", ["gffn_qwen3_t3", "gffn_tiny_t5"])
def test_qwen3_ffn_residual(name):
    """tie_hip_qwen3_ffn: RMSNorm (with the host RSQRTSS table), block and
    residual add, bit-exact against the oracle; against the compiled
    reference's vectors on the CPU they were made on."""
    g = load_golden(name)
    layer = golden_layer(g)
    k, eps = int(g["k"]), float(g["eps"])
    print("qwen3 ffn case %s" % name, flush=True)
    h, idx, w = tie_amd.qwen3_ffn(g["hidden"], layer, k, g["ffn_norm"], eps)
    rh, ri, rw = bind.qwen3_ffn(layer, g["hidden"], k, g["ffn_norm"], eps)
    assert_same(idx, ri, "topk_idx")
    assert_same(w, rw, "topk_w")
    assert_same(h, rh, "hidden")
    if golden_host_check(g):
        assert_same(h, g["hidden_out"], "golden hidden")


@pytest.mark.parametrize("T,flags", [(32, None), (200, "mfma")])
def test_qwen3_ffn_residual_device(T, flags):
    """Layer.forward_residual on device memory, in place (and out of place
    on a second call, which must give the same bits): the exact path
    bit-exact, the MFMA path with exact routing and bf16-bounded outputs."""
    import torch
    c = synth.CONFIGS["30b_t32"]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], None)
    hidden = synth.make_input(c["seed"] + T, T, c["d"]) * np.float32(3.0)
    norm = synth.make_norm_weight(c["seed"], c["d"])
    L = tie_amd.Layer.from_synth(layer)
    mode = tie_amd.PATH_MFMA if flags else tie_amd.PATH_EXACT
    hin = torch.from_numpy(hidden).cuda()
    hout = torch.empty_like(hin)
    L.forward_residual(hin, torch.from_numpy(norm).cuda(), 1e-6, T, 8, hout, flags=mode)
    hd = torch.from_numpy(hidden).cuda()
    nd = torch.from_numpy(norm).cuda()
    idx = torch.empty((T, 8), dtype=torch.int32, device="cuda")
    w = torch.empty((T, 8), dtype=torch.float32, device="cuda")
    print("residual device case T=%d %s" % (T, flags), flush=True)
    L.forward_residual(hd, nd, 1e-6, T, 8, None, idx, w, flags=tie_amd.PATH_MFMA if flags else tie_amd.PATH_EXACT)
    torch.cuda.synchronize()
    rh, ri, rw = bind.qwen3_ffn(layer, hidden, 8, norm, 1e-6)
    assert_same(idx.cpu().numpy(), ri, "topk_idx")
    assert_same(w.cpu().numpy(), rw, "topk_w")
    got = hd.cpu().numpy()
    assert_same(hout.cpu().numpy(), got, "out of place vs in place")
    assert_same(hin.cpu().numpy(), hidden, "input untouched out of place")
    if flags:
        d_got, d_want = got - hidden, rh - hidden  # the block's contribution
        e = float(np.linalg.norm(d_got - d_want) / np.linalg.norm(d_want))
        print("residual MFMA rel L2 of the block output %.3g" % e, flush=True)
        assert e <= 4e-3
    else:
        assert_same(got, rh, "hidden")
    L.close()


@pytest.mark.parametrize("name,literal", [("g30b_bf16_zipf_t4", False), ("g30b_bf16_zipf_literal_t4", True)])
def test_golden_bf16_zipf_device_api(name, literal):
    import torch
    g = load_golden(name)
    s = golden_layer(g)
    k = int(g["k"])
    L = tie_amd.Layer.from_synth(s, literal_bf16_stride=literal)
    x = torch.from_numpy(g["x"]).cuda()
    T = x.shape[0]
    out = torch.empty_like(x)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    L.forward(x, T, k, out, idx, w, flags=tie_amd.PATH_EXACT)
    torch.cuda.synchronize()
    ro, ri, rw = bind.moe_block(s, g["x"], k, literal_bf16_stride=literal)
    assert_same(idx.cpu().numpy(), ri, "topk_idx")
    assert_same(w.cpu().numpy(), rw, "topk_w")
    assert_same(out.cpu().numpy(), ro, "out")
    assert_same(idx.cpu().numpy(), g["topk_idx"], "golden topk_idx")
    L.close()


@pytest.mark.parametrize("cfg", ["30b_t1", "30b_t8", "30b_t32", "235b_t1", "lfm2_t1", "lfm2_t32"])
def test_full_size_configs(cfg):
    c = synth.CONFIGS[cfg]
    layer = synth_layer(c["seed"], c["d"], c["F"], c["E"], c["gu_type"], c["down_type"], c["zipf"],
                        c.get("routing", 0), c.get("probs_bias"))
    x = synth.make_input(c["seed"], c["T"], c["d"])
    run_both(layer, x, c["k"])


@pytest.mark.parametrize("gu,dn", [(synth.Q4_K, synth.Q6_K), (synth.Q6_K, synth.Q4_K), (synth.Q4_K, synth.Q4_K)])
def test_one_launch_forms_agree(gu, dn):
    """Both forms of the one-launch one-token kernel give TIE's bits: a lane
    per (row, block) dot, and lane pairs (each lane half of a block's
    accumulators and code words, lane 0 gathering the other half)."""
    layer = synth_layer(31, 1024, 768, 64, gu, dn, None)
    try:
        for form in (0, 1):
            tie_amd.debug_decode_form(form)
            print("one-launch form %d" % form, flush=True)
            run_both(layer, synth.make_input(32 + form, 1, 1024), 8)
    finally:
        tie_amd.debug_decode_form(-1)


@pytest.mark.parametrize("gu,dn", [(synth.BF16, synth.BF16), (synth.Q4_K, synth.BF16), (synth.BF16, synth.Q6_K)])
def test_one_token_other_types(gu, dn):
    """One token with BF16 on either side: routing in the gate/up prologue
    with a one-pair grouping (BF16 gate/up), or the separate grouping
    kernel."""
    layer = synth_layer(26, 512, 256, 32, gu, dn, None)
    for k in (1, 8):
        run_both(layer, synth.make_input(26 + k, 1, 512), k)


def test_ragged_token_counts_and_k():
    layer = synth_layer(21, 512, 512, 24, synth.Q4_K, synth.Q6_K, None)
    for T, k in [(1, 1), (3, 2), (5, 7), (9, 24), (13, 8)]:
        x = synth.make_input(21 + T, T, 512)
        run_both(layer, x, k)


@pytest.mark.parametrize("E", [200, 1024])
def test_wide_expert_counts(E):
    """Selection over more than 128 experts (several logits per lane, E not
    a multiple of 64), on the grouping kernel (T*k <= 4096) and on the
    separate selection + dispatch kernels (T*k > 4096)."""
    import torch
    layer = synth_layer(24 + E, 256, 256, E, synth.Q4_K, synth.Q6_K, None)
    for T, k in [(1, 8), (5, 32), (40, 8)]:
        x = synth.make_input(24 + T, T, 256)
        run_both(layer, x, k)
    T, k = 160, 32
    x = synth.make_input(25, T, 256)
    L = tie_amd.Layer.from_synth(layer)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    print("case E=%d T=%d k=%d forced exact" % (E, T, k), flush=True)
    L.forward(xd, T, k, out, idx, w, flags=tie_amd.PATH_EXACT)
    torch.cuda.synchronize()
    ro, ri, rw = bind.moe_block(layer, x, k)
    assert_same(idx.cpu().numpy(), ri, "topk_idx")
    assert_same(w.cpu().numpy(), rw, "topk_w")
    assert_same(out.cpu().numpy(), ro, "out")
    L.close()


def test_zero_tokens_and_nan_rows():
    layer = synth_layer(22, 256, 256, 16, synth.Q4_K, synth.Q6_K, None)
    out, idx, w = tie_amd.moe_ffn(np.zeros((0, 256), np.float32), layer, 4)
    assert out.shape == (0, 256)
    x = synth.make_input(22, 3, 256)
    x[1, 7] = np.nan  # NaN logits: no expert enters the top-k
    out, idx, w = tie_amd.moe_ffn(x, layer, 4)
    ro, ri, rw = bind.moe_block(layer, x, 4)
    assert_same(idx, ri, "topk_idx")
    assert (idx[1] == -1).all()
    assert_same(out[[0, 2]], ro[[0, 2]], "out")
    assert (out[1] == 0).all() and (ro[1] == 0).all()


def test_repeat_calls_are_identical():
    layer = synth_layer(23, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None)
    x = synth.make_input(23, 2, 2048)
    a = tie_amd.moe_ffn(x, layer, 8)
    for _ in range(3):
        b = tie_amd.moe_ffn(x, layer, 8)
        for p, q in zip(a, b):
            assert_same(p, q, "repeat")


def test_argument_errors_and_injected_oom():
    layer = synth_layer(24, 256, 256, 16, synth.Q4_K, synth.Q6_K, None)
    x = synth.make_input(24, 2, 256)
    with pytest.raises(tie_amd.TieError) as e:
        tie_amd.moe_ffn(x, layer, 17)  # k > E
    assert e.value.code == tie_amd.EINVAL
    lib = tie_amd.lib()
    rc = lib.tie_hip_moe_ffn(x.ctypes.data, 2, 250, 256, 16, 4, layer.router.ctypes.data, 0, layer.gate.ctypes.data,
                             12, layer.up.ctypes.data, 12, layer.down.ctypes.data, 14, x.ctypes.data, None, None)
    assert rc == tie_amd.EINVAL and "multiples of 256" in tie_amd.last_error()
    rc = lib.tie_hip_moe_ffn(x.ctypes.data, 2, 256, 256, 16, 4, layer.router.ctypes.data, 0, layer.gate.ctypes.data,
                             3, layer.up.ctypes.data, 3, layer.down.ctypes.data, 14, x.ctypes.data, None, None)
    assert rc == tie_amd.EINVAL
    other = synth_layer(25, 256, 256, 16, synth.Q4_K, synth.Q6_K, None)
    lib.tie_hip_debug_fail_alloc(1)
    with pytest.raises(tie_amd.TieError) as e:
        tie_amd.moe_ffn(x, other, 4)  # first call uploads: that allocation fails
    assert e.value.code == tie_amd.ENOMEM
    run_both(other, x, 4)  # and the library recovers


def test_gguf_model_load(tmp_path):
    """tie_hip_gguf_load: a qwen3moe file's layers run the FFN half
    (RMSNorm with the file's ffn_norm, block, residual) bit-exact against the
    oracle on the same tensors; an lfm2 file's layer routes by sigmoid with
    its exp_probs_b bias and skips the leading dense layers."""
    import torch
    from gguf_write import moe_model_file
    d, F, E, k, T = 512, 256, 16, 4, 6
    layers = [synth.make_layer(70 + i, d, F, E, synth.Q4_K, synth.Q6_K) for i in range(2)]
    norms = [synth.make_norm_weight(70 + i, d) for i in range(2)]
    p = str(tmp_path / "q.gguf")
    moe_model_file(p, "qwen3moe", layers, d, F, E, k, eps=1e-6, norms=norms)
    M = tie_amd.Model(p)
    assert (M.info.n_layers, M.info.routing) == (2, tie_amd.ROUTE_SOFTMAX)
    for n in range(2):
        hidden = synth.make_input(80 + n, T, d) * np.float32(2.0)
        hd = torch.from_numpy(hidden).cuda()
        print("gguf qwen3moe layer %d" % n, flush=True)
        M.layer(n).forward_residual(hd, M.ffn_norm(n), M.info.norm_eps, T, k, None, flags=tie_amd.PATH_EXACT)
        torch.cuda.synchronize()
        rh, _, _ = bind.qwen3_ffn(layers[n], hidden, k, norms[n], float(M.info.norm_eps))
        assert_same(hd.cpu().numpy(), rh, "gguf layer %d hidden" % n)
    M.close()

    lay = synth.make_layer(75, d, F, E, synth.Q4_K, synth.Q6_K, routing=1, probs_bias=0.05)
    p2 = str(tmp_path / "l.gguf")
    moe_model_file(p2, "lfm2", [lay], d, F, E, k, pbias=[lay.probs_bias], lead=1)
    M = tie_amd.Model(p2)
    assert M.layer(0) is None and M.layer(1) is not None
    x = synth.make_input(85, T, d)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    print("gguf lfm2 layer 1", flush=True)
    M.layer(1).forward(xd, T, k, out, idx, w, flags=tie_amd.PATH_EXACT)
    torch.cuda.synchronize()
    ro, ri, rw = bind.moe_block(lay, x, k)
    assert_same(idx.cpu().numpy(), ri, "lfm2 topk_idx")
    assert_same(w.cpu().numpy(), rw, "lfm2 topk_w")
    assert_same(out.cpu().numpy(), ro, "lfm2 out")
    M.close()


def test_one_token_nan_row_and_residual():
    """One token (the decode kernels): a NaN input selects no expert (output
    0); the residual form at T = 1 in place and out of place."""
    import torch
    layer = synth_layer(23, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None)
    x = synth.make_input(27, 1, 2048)
    x[0, 11] = np.nan
    out, idx, w = tie_amd.moe_ffn(x, layer, 8)
    ro, ri, rw = bind.moe_block(layer, x, 8)
    assert_same(idx, ri, "topk_idx")
    assert (idx == -1).all() and (out == 0).all() and (ro == 0).all()
    hidden = synth.make_input(28, 1, 2048) * np.float32(2.0)
    norm = synth.make_norm_weight(28, 2048)
    rh, ri, rw = bind.qwen3_ffn(layer, hidden, 8, norm, 1e-6)
    L = tie_amd.Layer.from_synth(layer)
    hd = torch.from_numpy(hidden).cuda()
    nd = torch.from_numpy(norm).cuda()
    hout = torch.empty_like(hd)
    idx_d = torch.empty((1, 8), dtype=torch.int32, device="cuda")
    w_d = torch.empty((1, 8), dtype=torch.float32, device="cuda")
    L.forward_residual(hd, nd, 1e-6, 1, 8, hout, idx_d, w_d)
    L.forward_residual(hd, nd, 1e-6, 1, 8)  # in place
    torch.cuda.synchronize()
    assert_same(idx_d.cpu().numpy(), ri, "topk_idx")
    assert_same(w_d.cpu().numpy(), rw, "topk_w")
    assert_same(hout.cpu().numpy(), rh, "out of place")
    assert_same(hd.cpu().numpy(), rh, "in place")
    L.close()


def test_workspace_per_caller_stream():
    """Forwards on two caller streams (not the library's), each growing its
    own workspace while the other stream's work may still be in flight:
    every result equals the oracle.  (Each stream keeps its own scratch;
    growing one drains the device before the old buffer is freed.)"""
    import torch
    layer = synth_layer(29, 512, 512, 16, synth.Q4_K, synth.Q6_K, None)
    L = tie_amd.Layer.from_synth(layer)
    k = 4
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cases = []
    for i, T in enumerate([3, 40, 150, 1, 300, 9]):  # growing and shrinking T per stream
        s = streams[i % 2]
        x = synth.make_input(29 + i, T, 512)
        with torch.cuda.stream(s):
            xd = torch.from_numpy(x).to("cuda", non_blocking=False)
            out = torch.empty_like(xd)
            idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
            w = torch.empty((T, k), dtype=torch.float32, device="cuda")
        s.synchronize()
        flags = tie_amd.PATH_MFMA if T > 64 else tie_amd.PATH_EXACT
        print("stream case %d T=%d" % (i, T), flush=True)
        L.forward(xd, T, k, out, idx, w, flags=flags, stream=s.cuda_stream)
        cases.append((x, out, idx, w, flags))
    torch.cuda.synchronize()
    for x, out, idx, w, flags in cases:
        ro, ri, rw = bind.moe_block(layer, x, k)
        assert_same(idx.cpu().numpy(), ri, "topk_idx")
        assert_same(w.cpu().numpy(), rw, "topk_w")
        got = out.cpu().numpy()
        if flags == tie_amd.PATH_EXACT:
            assert_same(got, ro, "out")
        else:
            assert float(np.linalg.norm(got - ro) / np.linalg.norm(ro)) <= 1e-3
    # releasing a stream's workspace: the next forward on it grows a new one
    for s in streams:
        tie_amd.stream_release(s.cuda_stream)
    x, out, idx, w, _ = cases[0]
    L.forward(torch.from_numpy(x).cuda(), 3, k, out, idx, w, flags=tie_amd.PATH_EXACT, stream=streams[0].cuda_stream)
    torch.cuda.synchronize()
    assert_same(out.cpu().numpy(), bind.moe_block(layer, x, k)[0], "after release")
    L.close()


def test_one_token_repeat_calls_and_types():
    """One-token forwards (router, then the decode gate/up and down+combine
    kernels) many times in a row, for both routings and mixed types:
    bit-exact against the oracle every time."""
    cases = [(synth_layer(23, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None), 8),
             (synth_layer(41, 512, 256, 32, synth.Q6_K, synth.Q4_K, None), 4),
             (synth_layer(42, 512, 512, 24, synth.Q4_K, synth.Q6_K, None, 1, 0.05), 6)]
    for n, (layer, k) in enumerate(cases):
        for rep in range(3):
            x = synth.make_input(50 + rep, 1, layer.d)
            print("one-token case %d rep %d" % (n, rep), flush=True)
            run_both(layer, x, k)


def test_one_token_graph_replays():
    """One-token forwards captured in a HIP graph (three forwards on three
    layers) and replayed with eager work in between: every replay equals
    the eager result bit for bit."""
    import torch
    layers = [synth_layer(60 + i, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None) for i in range(3)]
    Ls = [tie_amd.Layer.from_synth(l) for l in layers]
    xs = [torch.from_numpy(synth.make_input(61 + i, 1, 2048)).cuda() for i in range(3)]
    outs = [torch.empty_like(x) for x in xs]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for L, x, o in zip(Ls, xs, outs):
            L.forward(x, 1, 8, o, stream=s.cuda_stream)
    torch.cuda.synchronize()
    eager = [o.cpu().numpy() for o in outs]
    for i, l in enumerate(layers):
        ro, _, _ = bind.moe_block(l, xs[i].cpu().numpy(), 8)
        assert_same(eager[i], ro, "eager vs oracle")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        for L, x, o in zip(Ls, xs, outs):
            L.forward(x, 1, 8, o, stream=s.cuda_stream)
    for rep in range(4):
        for o in outs:
            o.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print("graph replay %d" % rep, flush=True)
        for i, o in enumerate(outs):
            assert_same(o.cpu().numpy(), eager[i], "replay %d layer %d" % (rep, i))
        # eager forwards between replays, on the library stream
        tie_amd.moe_ffn(xs[rep % 3].cpu().numpy(), layers[rep % 3], 8)
    del g
    for L in Ls:
        L.close()


@pytest.mark.gpu
def test_one_launch_back_to_back():
    """Eager one-token forwards (the one-launch kernel: router, gate/up and
    down workgroups handing over through sequence-stamped words) queued
    back to back on one stream over three layers with no synchronisation in
    between, then checked: each equals the oracle bit for bit, so no call
    read a word left by the call before it."""
    import torch
    cases = [(synth_layer(70, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None), 8),
             (synth_layer(71, 512, 256, 32, synth.Q6_K, synth.Q4_K, None), 4),
             (synth_layer(72, 4096, 1536, 128, synth.Q4_K, synth.Q6_K, None), 8)]
    Ls = [tie_amd.Layer.from_synth(l) for l, _ in cases]
    runs = []
    tie_amd.profile_enable(True)
    for i in range(12):
        c = i % 3
        layer, k = cases[c]
        x = torch.from_numpy(synth.make_input(80 + i, 1, layer.d)).cuda()
        out = torch.empty_like(x)
        idx = torch.empty((1, k), dtype=torch.int32, device="cuda")
        w = torch.empty((1, k), dtype=torch.float32, device="cuda")
        Ls[c].forward(x, 1, k, out, idx, w)
        runs.append((c, x, out, idx, w))
    torch.cuda.synchronize()
    prof = tie_amd.profile_read()
    tie_amd.profile_enable(False)
    assert prof.get("decode_one", (0, 0))[1] == 12, prof
    for i, (c, x, out, idx, w) in enumerate(runs):
        layer, k = cases[c]
        print("back-to-back call %d (layer %d)" % (i, c), flush=True)
        ro, ri, rw = bind.moe_block(layer, x.cpu().numpy(), k)
        assert_same(idx.cpu().numpy(), ri, "topk_idx")
        assert_same(w.cpu().numpy(), rw, "topk_w")
        assert_same(out.cpu().numpy(), ro, "out")
    for L in Ls:
        L.close()


@pytest.mark.gpu
def test_one_launch_give_up_is_reported():
    """A wait of the one-launch decode that gives up is reported, not just
    turned into NaN outputs: forced from the host (the debug hook makes the
    next call wait for a stamp no workgroup writes, with a 64-poll limit, so
    every workgroup still exits), the synchronous drop-in returns
    TIE_HIP_EHIP, and on the device API the outputs are NaN and
    tie_hip_stream_status raises once.  The calls after it are bit-exact."""
    import torch
    layer, k = synth_layer(73, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None), 8
    x = synth.make_input(90, 1, layer.d)
    ro, ri, rw = bind.moe_block(layer, x, k)
    print("give-up: host drop-in", flush=True)
    tie_amd.debug_decode_give_up(1)
    with pytest.raises(tie_amd.TieError) as ei:
        tie_amd.moe_ffn(x, layer, k)
    assert ei.value.code == tie_amd.EHIP and "gave up" in str(ei.value)
    out, idx, w = tie_amd.moe_ffn(x, layer, k)
    assert_same(out, ro, "after give-up (host)")
    print("give-up: device API", flush=True)
    L = tie_amd.Layer.from_synth(layer)
    s = torch.cuda.Stream()
    xd = torch.from_numpy(x).cuda()
    od = torch.empty_like(xd)
    tie_amd.debug_decode_give_up(1)
    L.forward(xd, 1, k, od, stream=s.cuda_stream)
    with pytest.raises(tie_amd.TieError) as ei:
        tie_amd.stream_status(s.cuda_stream)
    assert ei.value.code == tie_amd.EHIP
    assert np.isnan(od.cpu().numpy()).all()
    tie_amd.stream_status(s.cuda_stream)  # reported once
    L.forward(xd, 1, k, od, stream=s.cuda_stream)
    tie_amd.stream_status(s.cuda_stream)
    assert_same(od.cpu().numpy(), ro, "after give-up (device)")
    L.close()
