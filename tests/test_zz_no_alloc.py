"""tie_hip_moe_forward_noalloc (the entry point that allocates nothing: its
scratch is the library's static device array) against tie_hip_moe_forward
on the same inputs: identical selection and outputs, bit for bit (same
kernels, same arithmetic), on two calls in a row -- the second with fewer
tokens, so it runs on what the first left in the shared array -- on the
exact, one-token and matrix-core paths; sizes beyond the array are
refused."""
import numpy as np
import pytest

import tie_amd
from conftest import bits, synth_layer
from tie_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    import torch
    assert torch.cuda.is_available(), "GPU test without a GPU"
    tie_amd.init(0)
    yield
    tie_amd.shutdown()


def run(L, x, k, flags, noalloc):
    import torch
    T = x.shape[0]
    xd = torch.from_numpy(x).cuda()
    out = torch.full_like(xd, -7.0)
    idx = torch.full((T, k), -9, dtype=torch.int32, device="cuda")
    w = torch.full((T, k), -9.0, dtype=torch.float32, device="cuda")
    print("no-alloc case T=%d k=%d flags=%d noalloc=%d" % (T, k, flags, noalloc), flush=True)
    if noalloc:
        L.forward_noalloc(xd, T, k, out, idx, w, flags=flags)
    else:
        L.forward(xd, T, k, out, idx, w, flags=flags)
    torch.cuda.synchronize()
    return out.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()


# (PATH_MFMA, (32, 9)): the no-allocation scratch keeps the scanned tile
# list where the forward's workspace runs one item per (expert, slab) with
# h by expert -- the two give the same bits
@pytest.mark.parametrize("flags,Ts", [(tie_amd.PATH_EXACT, (40, 7)), (tie_amd.PATH_AUTO, (1, 1)),
                                      (tie_amd.PATH_MFMA, (80, 33)), (tie_amd.PATH_MFMA, (32, 9))])
def test_noalloc_matches_forward(flags, Ts):
    layer = synth_layer(71, 2048, 768, 128, synth.Q4_K, synth.Q6_K, None)
    L = tie_amd.Layer.from_synth(layer)
    k = 8
    xs = [synth.make_input(72 + T, T, 2048) for T in Ts]
    got = [run(L, x, k, flags, True) for x in xs]  # two no-alloc calls in a row, the second smaller
    for x, g in zip(xs, got):
        want = run(L, x, k, flags, False)
        for a, b, what in zip(g, want, ("out", "topk_idx", "topk_w")):
            np.testing.assert_array_equal(bits(a), bits(b), err_msg=what)
    L.close()


def test_noalloc_refuses_oversized_calls():
    import torch
    layer = synth_layer(73, 512, 512, 16, synth.Q4_K, synth.Q6_K, None)
    L = tie_amd.Layer.from_synth(layer)
    T = 20000
    xd = torch.zeros((T, 512), device="cuda")
    out = torch.empty_like(xd)
    with pytest.raises(tie_amd.TieError) as e:
        L.forward_noalloc(xd, T, 4, out)
    assert e.value.code == tie_amd.EINVAL and "scratch" in str(e.value)
    L.close()
