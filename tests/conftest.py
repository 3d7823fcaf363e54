import functools
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@functools.lru_cache(maxsize=None)
def synth_layer(seed, d, F, E, gu, dn, zipf, routing=0, probs_bias=None):
    from tie_amd import synth
    return synth.make_layer(seed, d, F, E, gu, dn, zipf=zipf, routing=routing, probs_bias=probs_bias)


def golden_layer(g):
    """Regenerate the weights of a golden case (cached per session)."""
    import copy
    zipf = float(g["zipf"]) or None
    routing = int(g["routing"]) if "routing" in g else 0
    pb = float(g["probs_bias"]) if "probs_bias" in g else 0.0
    layer = synth_layer(int(g["seed"]), int(g["d"]), int(g["F"]), int(g["E"]), int(g["gu_type"]),
                        int(g["down_type"]), zipf, routing, pb or None)
    ties = g["tie_rows"].reshape(-1, 2)
    sat = g["sat_rows"] if "sat_rows" in g else np.zeros(0, np.int32)
    if len(ties) or len(sat):
        layer = copy.copy(layer)
        layer.router = layer.router.copy()
        for a, b in ties:
            layer.router[b] = layer.router[a]
        for r in sat:
            layer.router[r] *= np.float32(100.0)
    return layer


def host_cpu_identity():
    from oracle import bind
    vendor = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("vendor_id"):
                    vendor = line.split(":")[1].strip()
                    break
    except OSError:
        pass
    import platform
    mode = bind.oracle().orc_silu_rcp_mode()
    return "%s/%s/rcp%s" % (vendor, platform.machine(), "14" if mode == 2 else "ps")


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a
