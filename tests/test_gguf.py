"""The GGUF reader of the library (tie_hip_gguf_inspect) on files written by
tests/gguf_write.py: metadata, architecture-dependent routing, and the
errors for malformed files.  Host only."""
import os

import numpy as np
import pytest

import tie_amd
from gguf_write import STR, U32, moe_model_file, write_gguf
from tie_amd import synth


def small_layers(n, d=256, F=256, E=8):
    return [synth.make_layer(60 + i, d, F, E, synth.Q4_K, synth.Q6_K) for i in range(n)]


def test_inspect_qwen3moe(tmp_path):
    p = str(tmp_path / "q.gguf")
    moe_model_file(p, "qwen3moe", small_layers(2), 256, 256, 8, 2, eps=1e-5)
    info = tie_amd.gguf_inspect(p)
    assert info.architecture == b"qwen3moe"
    assert (info.d, info.F, info.E, info.k, info.n_layers, info.first_moe_layer) == (256, 256, 8, 2, 2, 0)
    assert info.routing == tie_amd.ROUTE_SOFTMAX
    assert info.norm_eps == np.float32(1e-5)


def test_inspect_lfm2_leading_dense(tmp_path):
    p = str(tmp_path / "l.gguf")
    moe_model_file(p, "lfm2", small_layers(1), 256, 256, 8, 2, lead=2)
    info = tie_amd.gguf_inspect(p)
    assert (info.n_layers, info.first_moe_layer, info.routing) == (3, 2, tie_amd.ROUTE_SIGMOID)


def test_inspect_errors(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + b"\0" * 40)
    with pytest.raises(tie_amd.TieError, match="bad magic"):
        tie_amd.gguf_inspect(str(bad))
    with pytest.raises(tie_amd.TieError, match="cannot open"):
        tie_amd.gguf_inspect(str(tmp_path / "missing.gguf"))
    p = str(tmp_path / "q.gguf")
    moe_model_file(p, "qwen3moe", small_layers(1), 256, 256, 8, 2)
    data = open(p, "rb").read()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(data[:len(data) - 4096])  # the last tensor runs past the end
    with pytest.raises(tie_amd.TieError, match="past the end of the file"):
        tie_amd.gguf_inspect(str(cut))
    nomoe = str(tmp_path / "dense.gguf")
    write_gguf(nomoe, {"general.architecture": (STR, "qwen3"), "qwen3.embedding_length": (U32, 256)}, [])
    with pytest.raises(tie_amd.TieError, match="missing MoE metadata"):
        tie_amd.gguf_inspect(nomoe)


@pytest.mark.skipif(not __import__("oracle.bind", fromlist=["x"]).ref_available(),
                    reason="reference build absent")
@pytest.mark.parametrize("arch,lead", [("qwen3moe", 0), ("lfm2moe", 1)])
def test_reader_matches_tie_parser(tmp_path, arch, lead):
    """The library's GGUF reader against TIE's own (gguf_model_parse with
    gguf_model_map_weights, gguf.c:892-1047, compiled in oracle/_ref) on the
    same files: every tensor's type, dimensions, data offset in the file and
    size (for the types the MoE path reads), the metadata the block needs,
    and the architecture.  The files hold an extra tensor of a type the MoE
    path never reads (Q8_0, as a real model's embeddings) and a ragged
    tensor size, so the data offsets are not all multiples of a block."""
    import struct
    from oracle import bind
    from gguf_write import F32
    d, F, E, k = 256, 256, 8, 2
    layers = small_layers(2, d, F, E)
    norms = [synth.make_norm_weight(70 + i, d) for i in range(2)]
    pbias = [np.random.default_rng(80 + i).normal(0, 0.05, E).astype(np.float32) for i in range(2)]
    p = str(tmp_path / "m.gguf")
    # general.basename: TIE's detect_architecture reads it (model.c:65-96)
    meta = {"general.architecture": (STR, arch), "general.basename": (STR, "Synthetic-MoE"),
            arch + ".embedding_length": (U32, d), arch + ".block_count": (U32, lead + 2), arch + ".expert_count": (U32, E),
            arch + ".expert_used_count": (U32, k), arch + ".expert_feed_forward_length": (U32, F),
            arch + ".attention.layer_norm_rms_epsilon": (F32, 1e-6)}
    if lead:
        meta[arch + ".leading_dense_block_count"] = (U32, lead)
    tensors = [("token_embd.weight", bytes(34 * 40), 8, (256 * 5, 1)),  # Q8_0: 34 B per 32 weights
               ("output_norm.weight", np.ones(7, np.float32).tobytes(), 0, (7,))]
    for i, L in enumerate(layers):
        n = lead + i
        tensors += [("blk.%d.ffn_gate_inp.weight" % n, L.router.tobytes(), 0, (d, E)),
                    ("blk.%d.ffn_gate_exps.weight" % n, L.gate.tobytes(), L.gate_type, (d, F, E)),
                    ("blk.%d.ffn_up_exps.weight" % n, L.up.tobytes(), L.up_type, (d, F, E)),
                    ("blk.%d.ffn_down_exps.weight" % n, L.down.tobytes(), L.down_type, (F, d, E)),
                    ("blk.%d.ffn_norm.weight" % n, norms[i].tobytes(), 0, (d,)),
                    ("blk.%d.exp_probs_b.bias" % n, pbias[i].tobytes(), 0, (E,))]
    write_gguf(p, meta, tensors)
    keys = [arch + s for s in (".embedding_length", ".block_count", ".expert_count", ".expert_used_count",
                               ".expert_feed_forward_length", ".attention.layer_norm_rms_epsilon",
                               ".leading_dense_block_count")]
    ref = bind.ref_gguf(p, keys)
    assert ref is not None, "TIE's parser rejected the file"
    assert ref["arch"] >= 0
    assert tie_amd.gguf_tensor_count(p) == len(ref["tensors"]) == len(tensors)
    for name, (rt, rne, roff, rbytes) in ref["tensors"].items():
        t, ne, off, nbytes = tie_amd.gguf_tensor_info(p, name)
        assert (t, ne, off) == (rt, rne, roff), name
        if t in (synth.F32, synth.Q4_K, synth.Q6_K, synth.BF16):
            assert nbytes == rbytes, name
        else:
            assert nbytes == 0, name  # not a type the MoE path reads
    info = tie_amd.gguf_inspect(p)
    u32 = {k2: struct.unpack("<I", v[:4])[0] for k2, v in ref["values"].items() if not k2.endswith("epsilon")}
    assert (info.d, info.n_layers, info.E, info.k, info.F) == tuple(
        u32[arch + s] for s in (".embedding_length", ".block_count", ".expert_count", ".expert_used_count",
                                ".expert_feed_forward_length"))
    assert info.first_moe_layer == u32.get(arch + ".leading_dense_block_count", 0)
    eps = struct.unpack("<f", ref["values"][arch + ".attention.layer_norm_rms_epsilon"][:4])[0]
    assert info.norm_eps == np.float32(eps)
    assert info.routing == (tie_amd.ROUTE_SIGMOID if arch.startswith("lfm2") else tie_amd.ROUTE_SOFTMAX)
