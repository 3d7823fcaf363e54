"""The C-ABI library without a GPU: it loads, exports what include/tie_hip.h
declares, builds TIE's SiLU table on the host, and reports errors without
exiting."""
import os
import re
import sys

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


C_CALLER = r"""
#include <stdio.h>
#include <stdint.h>
#include "tie_hip.h"

/* the call site INTEGRATION.md shows, reduced to what runs without a GPU:
 * every prototype used with TIE's own argument types */
int main(void)
{
	static float table[TIE_SILU_TABLE_SIZE];
	float in[2] = {0.0f, -1.5f}, out[2];
	tie_hip_model_info info;
	int32_t idx[8];
	float w[8];
	int rc;
	tie_hip_host_expf(in, out, 2);
	rc = tie_hip_silu_table_host(table, TIE_SILU_TABLE_SIZE);
	if (rc != TIE_HIP_OK || out[0] != 1.0f)
		return 1;
	/* no device: a clear error code, no exit */
	rc = tie_hip_moe_ffn(in, 0, 2048, 768, 128, 8, table, TIE_GGML_F32, table, TIE_GGML_Q4_K, table,
			     TIE_GGML_Q4_K, table, TIE_GGML_Q6_K, out, idx, w);
	if (rc != TIE_HIP_ENOINIT)
		return 2;
	rc = tie_hip_gguf_inspect("/nonexistent.gguf", &info);
	if (rc == TIE_HIP_OK)
		return 3;
	printf("%s\n", tie_hip_last_error());
	return 0;
}
"""


def test_header_compiles_as_c99_and_links(tmp_path):
    """A C translation unit compiled the way TIE compiles (gcc, C99, all
    warnings as errors) against include/tie_hip.h, linked with
    libtie_hip.so, and run: the prototypes INTEGRATION.md relies on are
    plain C and the library answers without a GPU."""
    import subprocess
    src = tmp_path / "caller.c"
    src.write_text(C_CALLER)
    exe = tmp_path / "caller"
    libdir = os.path.dirname(tie_amd.LIB_PATH)
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", os.path.join(ROOT, "include"),
           str(src), "-o", str(exe), "-L", libdir, "-ltie_hip", "-Wl,-rpath," + libdir]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)


REF_DIR = "/root/reference"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_DIR, "model_qwen3.c")),
                    reason="the reference sources are not present")
def test_integration_snippets_compile_against_tie_headers(tmp_path):
    """INTEGRATION.md's call-site snippets (engine_alloc set-up, the Qwen3 MoE
    branch model_qwen3.c:404-471, the FFN half :390-491, the LFM2 branch
    model_lfm2.c:414-497), pasted into functions shaped like TIE's own
    (oracle/callsite.c) and compiled with TIE's headers (struct TIEContext,
    Model, LayerWeights: main.h, model.h:170-253, engine.h:36-125) and TIE's
    warning flags as errors: every argument type-checks against TIE's
    structures.  A snippet with one argument of the wrong type must fail to
    compile, so the check has teeth."""
    import subprocess
    inc = tmp_path / "inc"
    inc.mkdir()
    r = subprocess.run([sys.executable, os.path.join(ROOT, "oracle", "extract_callsite.py"),
                        os.path.join(ROOT, "INTEGRATION.md"), str(inc)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    base = ["gcc", "-std=gnu99", "-Wall", "-Wno-pointer-sign", "-Wno-unused-label", "-funsigned-char", "-Werror",
            "-DTIE_USE_HIP", "-I", REF_DIR, "-I", os.path.join(ROOT, "include"), "-I", str(inc), "-c",
            os.path.join(ROOT, "oracle", "callsite.c"), "-o", str(tmp_path / "callsite.o")]
    r = subprocess.run(base, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    # negative control: TIE's ffn_norm Tensor where the snippet passes F
    q = (inc / "qwen3_moe.inc").read_text()
    assert "ctx->model->expert_ffn_dim" in q
    (inc / "qwen3_moe.inc").write_text(q.replace("ctx->model->expert_ffn_dim", "l->ffn_norm", 1))
    r = subprocess.run(base, capture_output=True, text=True)
    assert r.returncode != 0 and "qwen3_moe.inc" in r.stderr
