"""The C-ABI library without a GPU: it loads, exports what include/tie_hip.h
declares, builds TIE's SiLU table on the host, and reports errors without
exiting."""
import os
import re

import numpy as np
import pytest

import tie_amd
from conftest import ROOT, bits
from oracle import bind

pytestmark = pytest.mark.skipif(not os.path.exists(tie_amd.LIB_PATH), reason="libtie_hip.so not built")


def header_symbols():
    src = open(os.path.join(ROOT, "include", "tie_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(tie_hip_[a-z0-9_]+)\s*\(", src))


def test_every_declared_symbol_is_exported():
    declared = header_symbols()
    assert declared == set(tie_amd.EXPORTS)
    lib = tie_amd.lib()
    for name in declared:
        assert hasattr(lib, name), name


def test_library_is_built_for_gfx950_only():
    import subprocess
    out = subprocess.run(["/opt/rocm/bin/roc-obj-ls", tie_amd.LIB_PATH], capture_output=True, text=True)
    if out.returncode != 0:
        pytest.skip("roc-obj-ls unavailable")
    targets = set(re.findall(r"gfx\d+\w*", out.stdout))
    assert targets == {"gfx950"}, targets


def test_host_silu_table_equals_oracle_table():
    np.testing.assert_array_equal(bits(tie_amd.silu_table_host()), bits(bind.silu_table()))


def test_errors_without_init():
    lib = tie_amd.lib()
    x = np.zeros((1, 256), np.float32)
    rc = lib.tie_hip_moe_ffn(x.ctypes.data, 1, 256, 256, 8, 2, None, 0, None, 12, None, 12, None, 14,
                             x.ctypes.data, None, None)
    assert rc == tie_amd.ENOINIT
    assert "tie_hip_init" in tie_amd.last_error()
    assert lib.tie_hip_silu_table_host(x.ctypes.data, 17) == tie_amd.EINVAL


def test_exact_threshold_setter():
    lib = tie_amd.lib()
    old = lib.tie_hip_exact_max_tokens()
    lib.tie_hip_set_exact_max_tokens(5)
    assert lib.tie_hip_exact_max_tokens() == 5
    lib.tie_hip_set_exact_max_tokens(-3)
    assert lib.tie_hip_exact_max_tokens() == 0
    lib.tie_hip_set_exact_max_tokens(old)
