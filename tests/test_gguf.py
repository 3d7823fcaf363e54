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
    with pytest.raises(tie_amd.TieError, match="out of the file"):
        tie_amd.gguf_inspect(str(cut))
    nomoe = str(tmp_path / "dense.gguf")
    write_gguf(nomoe, {"general.architecture": (STR, "qwen3"), "qwen3.embedding_length": (U32, 256)}, [])
    with pytest.raises(tie_amd.TieError, match="missing MoE metadata"):
        tie_amd.gguf_inspect(nomoe)
