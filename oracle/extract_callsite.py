"""Writes the C call-site snippets of INTEGRATION.md into include files for
oracle/callsite.c (TEST INFRASTRUCTURE ONLY): the code a TIE maintainer
pastes is the code the harness compiles against TIE's own headers and runs.

    python3 extract_callsite.py INTEGRATION.md OUTDIR

Each ```c block is matched by the entry point it calls:
  init.inc        tie_hip_init / tie_hip_set_silu_table   (engine_alloc, engine.c:14-40)
  qwen3_moe.inc   tie_hip_moe_ffn                         (model_qwen3.c:404-471)
  qwen3_ffn.inc   tie_hip_qwen3_ffn                       (model_qwen3.c:390-491)
  lfm2_moe.inc    tie_hip_moe_ffn_lfm2                    (model_lfm2.c:414-497)
"""
import re
import sys

KEYS = [("init.inc", "tie_hip_init("), ("qwen3_ffn.inc", "tie_hip_qwen3_ffn("),
        ("lfm2_moe.inc", "tie_hip_moe_ffn_lfm2("), ("qwen3_moe.inc", "tie_hip_moe_ffn(")]


def main(md, outdir):
    text = open(md).read()
    blocks = re.findall(r"```c\n(.*?)```", text, re.S)
    found = {}
    for b in blocks:
        for name, key in KEYS:
            if key in b and name not in found:
                found[name] = b
                break
    missing = [n for n, _ in KEYS if n not in found]
    if missing:
        sys.exit("INTEGRATION.md: no C block for %s" % ", ".join(missing))
    for name, b in found.items():
        with open("%s/%s" % (outdir, name), "w") as f:
            f.write("/* generated from INTEGRATION.md by extract_callsite.py */\n" + b)


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
