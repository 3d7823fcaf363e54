"""ctypes bindings for the parity checkers (TEST INFRASTRUCTURE ONLY).

liboracle.so      -- the C restatement of TIE's MoE path (tie_oracle.c)
_ref/libtie_ref.so -- the reference's own sources + ref_driver.c

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  The product (tie_amd) never does.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtie_ref.so")
SILU_N = 8192

_P = ctypes.c_void_p
_I = ctypes.c_int


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle not built: run `make -C oracle` (or __graft_entry__.build())")
        lib = ctypes.CDLL(ORACLE_SO)
        lib.orc_fp16_to_fp32.restype = ctypes.c_float
        lib.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.orc_dot_f32.restype = ctypes.c_float
        lib.orc_dot_f32.argtypes = [_P, _P, _I]
        lib.orc_dot_q4k_block.restype = ctypes.c_float
        lib.orc_dot_q4k_block.argtypes = [_P, _P]
        lib.orc_dot_q6k_block.restype = ctypes.c_float
        lib.orc_dot_q6k_block.argtypes = [_P, _P]
        lib.orc_matvec.restype = _I
        lib.orc_matvec.argtypes = [_P, _P, _I, _I, _I, _P]
        lib.orc_silu_rcp_mode.restype = _I
        lib.orc_silu_table.restype = _I
        lib.orc_silu_table.argtypes = [_P, _I]
        lib.orc_swiglu.argtypes = [_P, _P, _I, _P]
        lib.orc_find_top_k.argtypes = [_P, _I, _I, _P, _P]
        lib.orc_softmax.argtypes = [_P, _I]
        lib.orc_moe_block.restype = _I
        lib.orc_moe_block.argtypes = [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _P,
                                      _P, _P, _P, _P, _I]
        lib.orc_sigmoid_route.argtypes = [_P, _I, _I, _P, _P, _P]
        lib.orc_dequant_q4k.argtypes = [_P, _I, _P]
        lib.orc_dequant_q6k.argtypes = [_P, _I, _P]
        lib.orc_expf_array.argtypes = [_P, _P, ctypes.c_size_t]
        lib.orc_rms_norm.argtypes = [_P, _P, _I, ctypes.c_float, _P]
        lib.orc_qwen3_ffn.restype = _I
        lib.orc_qwen3_ffn.argtypes = [_P, _I, _I, _I, _I, _I, _P, ctypes.c_float, _P, _P, _I, _P, _I, _P, _I, _P,
                                      _P, _P, _I]
        _oracle = lib
    return _oracle


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError("reference build absent: oracle/_ref/libtie_ref.so")
        lib = ctypes.CDLL(REF_SO)
        lib.ref_silu_table.restype = _I
        lib.ref_gguf_open.restype = _P
        lib.ref_gguf_open.argtypes = [ctypes.c_char_p]
        lib.ref_gguf_close.argtypes = [_P]
        lib.ref_gguf_info.argtypes = [_P, _P, _P, _P]
        lib.ref_gguf_tensor.argtypes = [_P, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t, _P, _P, _P, _P, _P]
        lib.ref_gguf_value.argtypes = [_P, ctypes.c_char_p, _P]
        lib.ref_silu_table.argtypes = [_P, _I]
        lib.ref_pool_threads.restype = _I
        lib.ref_rms_norm.restype = _I
        lib.ref_rms_norm.argtypes = [_P, _P, _I, ctypes.c_float, _P, _I]
        lib.ref_apply_residual.restype = _I
        lib.ref_apply_residual.argtypes = [_P, _P, _I, _I]
        lib.ref_moe_block.restype = _I
        lib.ref_moe_block.argtypes = [_P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _P,
                                      _P, _P, _P, _I]
        _ref = lib
    return _ref


def silu_table(mode=0):
    t = np.empty(SILU_N, np.float32)
    if oracle().orc_silu_table(_ptr(t), mode) != 0:
        raise RuntimeError("silu table mode %d not available on this host" % mode)
    return t


def moe_block(layer, x, k, silu_tab=None, literal_bf16_stride=False, nthreads=8, with_logits=False):
    """Oracle MoE block on host arrays.  Returns (out, topk_idx, topk_w[, logits])."""
    x = np.ascontiguousarray(x, np.float32)
    T, d = x.shape
    if silu_tab is None:
        silu_tab = silu_table()
    out = np.empty((T, d), np.float32)
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    logits = np.empty((T, layer.E), np.float32) if with_logits else None
    rc = oracle().orc_moe_block(_ptr(x), T, d, layer.F, layer.E, k, _ptr(layer.router), _ptr(layer.bias),
                                int(getattr(layer, "routing", 0)), _ptr(getattr(layer, "probs_bias", None)),
                                _ptr(layer.gate), layer.gate_type, _ptr(layer.up), layer.up_type,
                                _ptr(layer.down), layer.down_type, int(literal_bf16_stride), _ptr(silu_tab),
                                _ptr(out), _ptr(idx), _ptr(w), _ptr(logits), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the block shape/types")
    return (out, idx, w, logits) if with_logits else (out, idx, w)


def ref_moe_block(layer, x, k, literal_bf16_stride=False, nthreads=8, with_logits=False):
    """The compiled reference's MoE path on host arrays."""
    x = np.ascontiguousarray(x, np.float32)
    T, d = x.shape
    out = np.empty((T, d), np.float32)
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    logits = np.empty((T, layer.E), np.float32) if with_logits else None
    rc = ref().ref_moe_block(_ptr(x), T, d, layer.F, layer.E, k, _ptr(layer.router), _ptr(layer.bias),
                             int(getattr(layer, "routing", 0)), _ptr(getattr(layer, "probs_bias", None)),
                             _ptr(layer.gate), layer.gate_type, _ptr(layer.up), layer.up_type, _ptr(layer.down),
                             layer.down_type, int(literal_bf16_stride), _ptr(out), _ptr(idx), _ptr(w),
                             _ptr(logits), nthreads)
    if rc != 0:
        raise ValueError("reference driver failed")
    return (out, idx, w, logits) if with_logits else (out, idx, w)


def rms_norm(x, w, eps):
    """Oracle RMSNorm of every row of x (TIE's rms_norm with this host's RSQRTSS)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        oracle().orc_rms_norm(_ptr(x[t]), _ptr(w), x.shape[1], eps, _ptr(out[t]))
    return out


def ref_rms_norm(x, w, eps, nthreads=8):
    """The compiled reference's dispatch_rms_norm on every row of x."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        if ref().ref_rms_norm(_ptr(x[t]), _ptr(w), x.shape[1], eps, _ptr(out[t]), nthreads) != 0:
            raise RuntimeError("reference rms_norm failed")
    return out


def qwen3_ffn(layer, hidden, k, ffn_norm, eps, silu_tab=None, nthreads=8):
    """Oracle FFN half of the layer: hidden + block(rms_norm(hidden)).
    Returns (new hidden, topk_idx, topk_w); the input array is not changed."""
    h = np.array(hidden, np.float32, copy=True, order="C")
    T, d = h.shape
    if silu_tab is None:
        silu_tab = silu_table()
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    norm = np.ascontiguousarray(ffn_norm, np.float32)
    rc = oracle().orc_qwen3_ffn(_ptr(h), T, d, layer.F, layer.E, k, _ptr(norm), eps, _ptr(layer.router),
                                _ptr(layer.gate), layer.gate_type, _ptr(layer.up), layer.up_type, _ptr(layer.down),
                                layer.down_type, _ptr(silu_tab), _ptr(idx), _ptr(w), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the block shape/types")
    return h, idx, w


def mat_mat(x, w, wtype, rows):
    """Oracle dispatch_mat_mat with F32 input: every row of x through TIE's
    row kernel for the weight type."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((x.shape[0], rows), np.float32)
    for t in range(x.shape[0]):
        if oracle().orc_matvec(_ptr(x[t]), _ptr(w), wtype, x.shape[1], rows, _ptr(out[t])) != 0:
            raise ValueError("oracle rejected the matrix type")
    return out


def ref_silu_table(nthreads=8):
    t = np.empty(SILU_N, np.float32)
    if ref().ref_silu_table(_ptr(t), nthreads) != 0:
        raise RuntimeError("reference silu table failed")
    return t


def libm_expf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    oracle().orc_expf_array(_ptr(x), _ptr(out), x.size)
    return out


def ref_gguf(path, keys=()):
    """TIE's own GGUF reader (gguf_model_parse, gguf.c:968-1047) on a file:
    {"arch": id, "data_offset": .., "tensors": {name: (type, ne[4], file
    offset, bytes)}, "values": {key: 8 raw bytes}} (None if TIE rejects the
    file)."""
    import os
    lib = ref()
    h = lib.ref_gguf_open(os.fsencode(path))
    if not h:
        return None
    try:
        cnt, doff, arch = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_int()
        lib.ref_gguf_info(h, ctypes.byref(cnt), ctypes.byref(doff), ctypes.byref(arch))
        tensors = {}
        for i in range(cnt.value):
            name = ctypes.create_string_buffer(256)
            t, nd, off, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
            ne = np.zeros(4, np.uint64)
            lib.ref_gguf_tensor(h, i, name, 256, ctypes.byref(t), ctypes.byref(nd), _ptr(ne), ctypes.byref(off),
                                ctypes.byref(nb))
            tensors[name.value.decode()] = (t.value, tuple(int(v) for v in ne), off.value, nb.value)
        values = {}
        for k in keys:
            buf = (ctypes.c_uint8 * 8)()
            if lib.ref_gguf_value(h, k.encode(), buf) == 0:
                values[k] = bytes(buf)
        return {"arch": arch.value, "data_offset": doff.value, "tensors": tensors, "values": values}
    finally:
        lib.ref_gguf_close(h)
