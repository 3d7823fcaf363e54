"""A minimal GGUF v3 writer for the tests (test infrastructure): metadata
(u32, f32, string) and tensors laid out as TIE's loader reads them
(gguf.c:892-966): tensor data at the first multiple of the alignment after
the tensor infos, each tensor's offset aligned too."""
import struct

import numpy as np

U32, F32, STR = 4, 6, 8


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, meta, tensors, alignment=32):
    """meta: {key: (type, value)}; tensors: [(name, bytes-like, ggml type, ne tuple)]."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", 3, len(tensors), len(meta))
    for k, (t, v) in meta.items():
        out += _str(k) + struct.pack("<I", t)
        if t == U32:
            out += struct.pack("<I", v)
        elif t == F32:
            out += struct.pack("<f", v)
        elif t == STR:
            out += _str(v)
        else:
            raise ValueError(t)
    offs, off = [], 0
    for name, data, gtype, ne in tensors:
        offs.append(off)
        out += _str(name) + struct.pack("<I", len(ne)) + struct.pack("<%dQ" % len(ne), *ne)
        out += struct.pack("<IQ", gtype, off)
        off += len(bytes(data))
        off = (off + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (name, data, gtype, ne), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(bytes(out))


def moe_model_file(path, arch, layers, d, F, E, k, eps=1e-6, norms=None, pbias=None, lead=0):
    """A GGUF file with the MoE FFN tensors of `layers` (tie_amd.synth MoELayer,
    one per block from `lead` on) and optional ffn_norm / exp_probs_b."""
    meta = {"general.architecture": (STR, arch), arch + ".embedding_length": (U32, d),
            arch + ".block_count": (U32, lead + len(layers)), arch + ".expert_count": (U32, E),
            arch + ".expert_used_count": (U32, k), arch + ".expert_feed_forward_length": (U32, F),
            arch + ".attention.layer_norm_rms_epsilon": (F32, eps)}
    if lead:
        meta[arch + ".leading_dense_block_count"] = (U32, lead)
    tensors = []
    for i, L in enumerate(layers):
        n = lead + i
        tensors.append(("blk.%d.ffn_gate_inp.weight" % n, np.ascontiguousarray(L.router, np.float32).tobytes(), 0,
                        (d, E)))
        tensors.append(("blk.%d.ffn_gate_exps.weight" % n, L.gate.tobytes(), L.gate_type, (d, F, E)))
        tensors.append(("blk.%d.ffn_up_exps.weight" % n, L.up.tobytes(), L.up_type, (d, F, E)))
        tensors.append(("blk.%d.ffn_down_exps.weight" % n, L.down.tobytes(), L.down_type, (F, d, E)))
        if norms is not None:
            tensors.append(("blk.%d.ffn_norm.weight" % n, np.asarray(norms[i], np.float32).tobytes(), 0, (d,)))
        if pbias is not None:
            tensors.append(("blk.%d.exp_probs_b.bias" % n, np.asarray(pbias[i], np.float32).tobytes(), 0, (E,)))
    write_gguf(path, meta, tensors)
