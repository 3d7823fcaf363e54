"""Write the golden vectors of the MoE block from the compiled reference.

Run in a container that has the reference sources (oracle/Makefile builds
oracle/_ref/libtie_ref.so from them):

    make -C oracle && python tests/golden/make_golden.py

Each case regenerates its weights from tie_amd.synth (seeded) and stores
only what the reference computed from them -- router logits, selected
experts, gate weights and block outputs -- plus the SHA-256 of the weight
bytes, so a change in the generator is caught.  The SiLU table TIE builds
is stored with the host CPU's identity: its bits depend on the CPU's
approximate-reciprocal instruction (see oracle/tie_oracle.c).
"""
import os
import platform
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import bind  # noqa: E402
from tie_amd import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# name: (d, F, E, k, T, gate/up type, down type, zipf, seed, literal_bf16_stride, tie_rows[, lfm2])
# lfm2 = (probs_bias std or 0, rows scaled by 100): sigmoid routing (model_lfm2.c:437-467); the
# scaled rows give logits far outside [-20, 20], whose sigmoids saturate to
# 1.0 (or 0.0) and tie, exercising find_top_k's index order on equal p.
CASES = {
    "g30b_q4k_t4": (2048, 768, 128, 8, 4, synth.Q4_K, synth.Q6_K, None, 1234, 0, None),
    "g235b_e16_t2": (4096, 1536, 16, 8, 2, synth.Q4_K, synth.Q6_K, None, 1238, 0, None),
    "gtiny_q4k_t8": (256, 256, 16, 4, 8, synth.Q4_K, synth.Q6_K, None, 7, 0, None),
    "gtiny_q6k_q4k_t8": (512, 256, 16, 4, 8, synth.Q6_K, synth.Q4_K, None, 8, 0, None),
    "gtiny_ties_t6": (256, 256, 16, 4, 6, synth.Q4_K, synth.Q6_K, None, 9, 0, ((3, 5), (5, 11), (0, 1))),
    "g30b_bf16_zipf_t4": (2048, 768, 128, 8, 4, synth.BF16, synth.BF16, 1.2, 1237, 0, None),
    "g30b_bf16_zipf_literal_t4": (2048, 768, 128, 8, 4, synth.BF16, synth.BF16, 1.2, 1237, 1, None),
    "glfm2_t4": (2048, 1792, 32, 4, 4, synth.Q4_K, synth.Q6_K, None, 1250, 0, None, (0.05, ())),
    "glfm2_sat_t6": (512, 512, 32, 4, 6, synth.Q4_K, synth.Q6_K, None, 1252, 0, None, (0.0, (2, 9, 17, 30))),
}


def cpu_identity():
    vendor = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("vendor_id"):
                    vendor = line.split(":")[1].strip()
                    break
    except OSError:
        pass
    mode = bind.oracle().orc_silu_rcp_mode()
    return "%s/%s/rcp%s" % (vendor, platform.machine(), "14" if mode == 2 else "ps")


def build_case(name, spec):
    d, F, E, k, T, gu, dn, zipf, seed, literal, tie_rows = spec[:11]
    pb, sat = spec[11] if len(spec) > 11 else (None, ())
    lfm2 = len(spec) > 11
    layer = synth.make_layer(seed, d, F, E, gu, dn, zipf=zipf, routing=1 if lfm2 else 0, probs_bias=pb or None)
    if tie_rows:
        # identical router rows -> identical logits: exercises find_top_k's tie order
        for a, b in tie_rows:
            layer.router[b] = layer.router[a]
    for r in sat:
        layer.router[r] *= np.float32(100.0)
    x = synth.make_input(seed, T, d)
    out, idx, w, logits = bind.ref_moe_block(layer, x, k, literal_bf16_stride=bool(literal), with_logits=True)
    c = dict(name=name, d=d, F=F, E=E, k=k, T=T, gu_type=gu, down_type=dn, zipf=zipf or 0.0, seed=seed,
             literal=literal, tie_rows=np.array(tie_rows or [], np.int32).reshape(-1, 2),
             digest=layer.digest(), x=x, out=out, topk_idx=idx, topk_w=w, logits=logits,
             cpu=cpu_identity())
    if lfm2:
        c.update(routing=1, probs_bias=pb or 0.0, sat_rows=np.array(sat, np.int32))
    return c


# The FFN half of a Qwen3 layer through the compiled reference: RMSNorm of
# each token (dispatch_rms_norm), the MoE block, the residual add
# (dispatch_apply_residual).  name: (d, F, E, k, T, seed, eps)
FFN_CASES = {
    "gffn_qwen3_t3": (2048, 768, 128, 8, 3, 1260, 1e-6),
    "gffn_tiny_t5": (512, 256, 16, 4, 5, 1261, 1e-6),
}


def build_ffn_case(name, spec):
    d, F, E, k, T, seed, eps = spec
    layer = synth.make_layer(seed, d, F, E, synth.Q4_K, synth.Q6_K)
    hidden = synth.make_input(seed, T, d) * np.float32(3.0)
    norm = synth.make_norm_weight(seed, d)
    normed = bind.ref_rms_norm(hidden, norm, eps)
    out, idx, w = bind.ref_moe_block(layer, normed, k)
    new = hidden.copy()
    for t in range(T):
        if bind.ref().ref_apply_residual(bind._ptr(new[t]), bind._ptr(out[t]), d, 8) != 0:
            raise RuntimeError("reference residual failed")
    return dict(name=name, d=d, F=F, E=E, k=k, T=T, seed=seed, eps=np.float32(eps), gu_type=synth.Q4_K,
                down_type=synth.Q6_K, zipf=0.0, literal=0, tie_rows=np.zeros((0, 2), np.int32),
                digest=layer.digest(), hidden=hidden, ffn_norm=norm, normed=normed, hidden_out=new, topk_idx=idx,
                topk_w=w, cpu=cpu_identity())


def main():
    """python make_golden.py [case ...]: the named cases (default: all, and
    the SiLU table)."""
    names = sys.argv[1:] or list(CASES) + list(FFN_CASES)
    if not sys.argv[1:]:
        tab = bind.ref_silu_table()
        np.savez_compressed(os.path.join(OUT, "silu_table.npz"), table=tab, cpu=cpu_identity())
    for name in names:
        if name in FFN_CASES:
            c = build_ffn_case(name, FFN_CASES[name])
            np.savez_compressed(os.path.join(OUT, name + ".npz"), **c)
            print(name, "max|hidden_out| = %.4g" % np.abs(c["hidden_out"]).max())
            continue
        spec = CASES[name]
        c = build_case(name, spec)
        np.savez_compressed(os.path.join(OUT, name + ".npz"), **c)
        print(name, "max|out| = %.4g" % np.abs(c["out"]).max())


if __name__ == "__main__":
    main()
