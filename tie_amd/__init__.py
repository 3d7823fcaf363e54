"""tie_amd -- MI355X (gfx950) Qwen3-MoE FFN block for TIE.

The product is the C-ABI library ``libtie_hip.so`` (include/tie_hip.h),
built from tie_amd/csrc by tie_amd/Makefile.  This module is a thin ctypes
binding used by the tests and bench.py; it mirrors the C entry points one to
one and adds no computation of its own.  Importing it never falls back to a
CPU path: if the library is missing, every call raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TIE_AMD_LIB selects another build of the same library (e.g. a tuning variant)
LIB_PATH = os.environ.get("TIE_AMD_LIB") or os.path.join(HERE, "libtie_hip.so")

F32, Q4_K, Q6_K, BF16 = 0, 12, 14, 30
OK, EINVAL, EHIP, ENOMEM, ENOINIT = 0, -1, -2, -3, -4
PATH_AUTO, PATH_EXACT, PATH_MFMA = 0, 1, 2
ROUTE_SOFTMAX, ROUTE_SIGMOID = 0, 1
SILU_TABLE_SIZE = 8192

# every symbol include/tie_hip.h declares
EXPORTS = (
    "tie_hip_init", "tie_hip_shutdown", "tie_hip_last_error", "tie_hip_moe_ffn", "tie_hip_moe_ffn_lfm2",
    "tie_hip_qwen3_ffn", "tie_hip_moe_forward_residual", "tie_hip_matrix_create", "tie_hip_matrix_destroy",
    "tie_hip_mat_mat", "tie_hip_gguf_inspect", "tie_hip_gguf_tensor_info", "tie_hip_gguf_load", "tie_hip_model_info_get", "tie_hip_model_layer",
    "tie_hip_model_ffn_norm", "tie_hip_model_close", "tie_hip_set_silu_table",
    "tie_hip_silu_table_host", "tie_hip_layer_create", "tie_hip_layer_destroy", "tie_hip_layer_bytes",
    "tie_hip_moe_forward", "tie_hip_exact_max_tokens", "tie_hip_set_exact_max_tokens",
    "tie_hip_debug_fail_alloc", "tie_hip_host_expf", "tie_hip_profile_enable", "tie_hip_profile_read",
    "tie_hip_moe_forward_noalloc", "tie_hip_stream_status", "tie_hip_debug_decode_give_up", "tie_hip_debug_decode_form",
    "tie_hip_stream_release", "tie_hip_debug_layer_shifts",
)


class TieError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("tie_hip error %d: %s" % (code, msg))
        self.code = code


class LayerDesc(ctypes.Structure):
    _fields_ = [
        ("d", ctypes.c_int), ("F", ctypes.c_int), ("E", ctypes.c_int),
        ("router_w", ctypes.c_void_p), ("router_type", ctypes.c_int),
        ("gate_exps", ctypes.c_void_p), ("gate_type", ctypes.c_int),
        ("up_exps", ctypes.c_void_p), ("up_type", ctypes.c_int),
        ("down_exps", ctypes.c_void_p), ("down_type", ctypes.c_int),
        ("router_bias", ctypes.c_void_p),
        ("src_on_device", ctypes.c_int),
        ("literal_bf16_stride", ctypes.c_int),
        ("routing", ctypes.c_int),
        ("probs_bias", ctypes.c_void_p),
    ]


class ModelInfo(ctypes.Structure):
    _fields_ = [
        ("architecture", ctypes.c_char * 32),
        ("d", ctypes.c_int), ("F", ctypes.c_int), ("E", ctypes.c_int), ("k", ctypes.c_int),
        ("n_layers", ctypes.c_int), ("first_moe_layer", ctypes.c_int),
        ("norm_eps", ctypes.c_float), ("routing", ctypes.c_int),
    ]


_lib = None


def lib():
    """The loaded C-ABI library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libtie_hip.so is not built: run `make -C tie_amd` or __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        P, I = ctypes.c_void_p, ctypes.c_int
        L.tie_hip_init.argtypes = [I]
        L.tie_hip_init.restype = I
        L.tie_hip_shutdown.restype = None
        L.tie_hip_last_error.restype = ctypes.c_char_p
        L.tie_hip_moe_ffn.argtypes = [P, I, I, I, I, I, P, I, P, I, P, I, P, I, P, P, P]
        L.tie_hip_moe_ffn.restype = I
        L.tie_hip_moe_ffn_lfm2.argtypes = [P, I, I, I, I, I, P, I, P, P, I, P, I, P, I, P, P, P]
        L.tie_hip_moe_ffn_lfm2.restype = I
        L.tie_hip_qwen3_ffn.argtypes = [P, I, I, I, I, I, P, ctypes.c_float, P, I, P, I, P, I, P, I, P, P]
        L.tie_hip_qwen3_ffn.restype = I
        L.tie_hip_moe_forward_residual.argtypes = [P, P, P, ctypes.c_float, I, I, P, P, P, I, P]
        L.tie_hip_moe_forward_residual.restype = I
        L.tie_hip_matrix_create.argtypes = [P, I, I, I, I, ctypes.POINTER(ctypes.c_void_p)]
        L.tie_hip_matrix_create.restype = I
        L.tie_hip_matrix_destroy.argtypes = [P]
        L.tie_hip_matrix_destroy.restype = None
        L.tie_hip_mat_mat.argtypes = [P, P, I, P, I, P]
        L.tie_hip_mat_mat.restype = I
        L.tie_hip_gguf_inspect.argtypes = [ctypes.c_char_p, ctypes.POINTER(ModelInfo)]
        L.tie_hip_gguf_inspect.restype = I
        L.tie_hip_gguf_tensor_info.argtypes = [ctypes.c_char_p, ctypes.c_char_p, P, P, P, P]
        L.tie_hip_gguf_tensor_info.restype = I
        L.tie_hip_gguf_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
        L.tie_hip_gguf_load.restype = I
        L.tie_hip_model_info_get.argtypes = [P, ctypes.POINTER(ModelInfo)]
        L.tie_hip_model_info_get.restype = None
        L.tie_hip_model_layer.argtypes = [P, I]
        L.tie_hip_model_layer.restype = P
        L.tie_hip_model_ffn_norm.argtypes = [P, I]
        L.tie_hip_model_ffn_norm.restype = P
        L.tie_hip_model_close.argtypes = [P]
        L.tie_hip_model_close.restype = None
        L.tie_hip_set_silu_table.argtypes = [P, I]
        L.tie_hip_set_silu_table.restype = I
        L.tie_hip_silu_table_host.argtypes = [P, I]
        L.tie_hip_silu_table_host.restype = I
        L.tie_hip_layer_create.argtypes = [ctypes.POINTER(LayerDesc), ctypes.POINTER(ctypes.c_void_p)]
        L.tie_hip_layer_create.restype = I
        L.tie_hip_layer_destroy.argtypes = [P]
        L.tie_hip_layer_destroy.restype = None
        L.tie_hip_layer_bytes.argtypes = [P]
        L.tie_hip_layer_bytes.restype = ctypes.c_size_t
        L.tie_hip_moe_forward.argtypes = [P, P, I, I, P, P, P, I, P]
        L.tie_hip_moe_forward.restype = I
        L.tie_hip_moe_forward_noalloc.argtypes = [P, P, I, I, P, P, P, I, P]
        L.tie_hip_moe_forward_noalloc.restype = I
        L.tie_hip_exact_max_tokens.restype = I
        L.tie_hip_set_exact_max_tokens.argtypes = [I]
        L.tie_hip_set_exact_max_tokens.restype = None
        L.tie_hip_debug_fail_alloc.argtypes = [I]
        L.tie_hip_debug_fail_alloc.restype = None
        L.tie_hip_host_expf.argtypes = [P, P, ctypes.c_size_t]
        L.tie_hip_host_expf.restype = None
        L.tie_hip_debug_layer_shifts.argtypes = [P, P, P]
        L.tie_hip_debug_layer_shifts.restype = I
        L.tie_hip_stream_release.argtypes = [P]
        L.tie_hip_stream_release.restype = I
        L.tie_hip_stream_status.argtypes = [P]
        L.tie_hip_stream_status.restype = I
        L.tie_hip_debug_decode_give_up.argtypes = [I]
        L.tie_hip_debug_decode_give_up.restype = None
        L.tie_hip_debug_decode_form.argtypes = [I]
        L.tie_hip_debug_decode_form.restype = None
        L.tie_hip_profile_enable.argtypes = [I]
        L.tie_hip_profile_enable.restype = I
        L.tie_hip_profile_read.argtypes = [ctypes.c_char_p, ctypes.c_size_t, P, P, I]
        L.tie_hip_profile_read.restype = I
        _lib = L
    return _lib


def last_error():
    return lib().tie_hip_last_error().decode()


def check(rc):
    if rc != OK:
        raise TieError(rc, last_error())
    return rc


def _p(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data


def init(device=0):
    check(lib().tie_hip_init(device))


def shutdown():
    lib().tie_hip_shutdown()


def silu_table_host():
    t = np.empty(SILU_TABLE_SIZE, np.float32)
    check(lib().tie_hip_silu_table_host(_p(t), SILU_TABLE_SIZE))
    return t


def set_silu_table(table):
    table = np.ascontiguousarray(table, np.float32)
    check(lib().tie_hip_set_silu_table(_p(table), table.size))


def host_expf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().tie_hip_host_expf(_p(x), _p(out), x.size)
    return out


def stream_status(stream=None):
    """tie_hip_stream_status: raises TieError when a one-token forward on
    the stream had a wait between workgroups give up since the last check."""
    check(lib().tie_hip_stream_status(stream))


def stream_release(stream=None):
    """tie_hip_stream_release: free the workspace kept for the stream."""
    check(lib().tie_hip_stream_release(stream))


def debug_decode_give_up(n):
    lib().tie_hip_debug_decode_give_up(int(n))


def debug_decode_form(form):
    """Force the one-token kernel's form (0 a lane per dot, 1 lane pairs;
    -1 by the shape)."""
    lib().tie_hip_debug_decode_form(int(form))


def profile_enable(on=True):
    check(lib().tie_hip_profile_enable(int(on)))


def profile_read(max_kernels=32):
    """{kernel name: (total ms, launches)} since profile_enable(True)."""
    names = ctypes.create_string_buffer(4096)
    tot = np.zeros(max_kernels, np.float64)
    cnt = np.zeros(max_kernels, np.int32)
    n = lib().tie_hip_profile_read(names, 4096, _p(tot), _p(cnt), max_kernels)
    if n < 0:
        check(n)
    keys = names.value.decode().split(",") if n else []
    return {k: (float(tot[i]), int(cnt[i])) for i, k in enumerate(keys)}


def moe_ffn(x, layer, k, with_topk=True):
    """tie_hip_moe_ffn on host arrays (the drop-in for model_qwen3.c:404-471),
    or tie_hip_moe_ffn_lfm2 (model_lfm2.c:414-497) for a layer with sigmoid
    routing.  `layer` is a tie_amd.synth.MoELayer (GGUF-layout host arrays)."""
    x = np.ascontiguousarray(x, np.float32)
    T, d = x.shape
    out = np.empty((T, d), np.float32)
    idx = np.empty((T, k), np.int32) if with_topk else None
    w = np.empty((T, k), np.float32) if with_topk else None
    if layer.bias is not None:
        raise ValueError("the host drop-ins take no logit bias (TIE has none); use Layer for biased routing")
    if getattr(layer, "routing", ROUTE_SOFTMAX) == ROUTE_SIGMOID:
        # tie_hip_moe_ffn_lfm2: the drop-in for model_lfm2.c:414-497
        check(lib().tie_hip_moe_ffn_lfm2(_p(x), T, d, layer.F, layer.E, k, _p(layer.router), F32,
                                         _p(layer.probs_bias), _p(layer.gate), layer.gate_type, _p(layer.up),
                                         layer.up_type, _p(layer.down), layer.down_type, _p(out), _p(idx),
                                         _p(w)))
    else:
        check(lib().tie_hip_moe_ffn(_p(x), T, d, layer.F, layer.E, k, _p(layer.router), F32, _p(layer.gate),
                                    layer.gate_type, _p(layer.up), layer.up_type, _p(layer.down),
                                    layer.down_type, _p(out), _p(idx), _p(w)))
    return out, idx, w


def qwen3_ffn(hidden, layer, k, ffn_norm, eps, with_topk=True):
    """tie_hip_qwen3_ffn on host arrays: the FFN half of transformer_layer_qwen3
    (RMSNorm, MoE block, residual add; model_qwen3.c:392-491).  Returns the
    new hidden state (the input array is not changed) and the selection."""
    h = np.array(hidden, np.float32, copy=True, order="C")
    T, d = h.shape
    idx = np.empty((T, k), np.int32) if with_topk else None
    w = np.empty((T, k), np.float32) if with_topk else None
    norm = np.ascontiguousarray(ffn_norm, np.float32)
    check(lib().tie_hip_qwen3_ffn(_p(h), T, d, layer.F, layer.E, k, _p(norm), eps, _p(layer.router), F32,
                                  _p(layer.gate), layer.gate_type, _p(layer.up), layer.up_type, _p(layer.down),
                                  layer.down_type, _p(idx), _p(w)))
    return h, idx, w


def gguf_tensor_info(path, name):
    """tie_hip_gguf_tensor_info: (type, ne[4], file offset, bytes) of one
    tensor as the library's reader maps it (no GPU needed)."""
    t = ctypes.c_int(0)
    ne = np.zeros(4, np.uint64)
    off = ctypes.c_uint64(0)
    nb = ctypes.c_uint64(0)
    rc = lib().tie_hip_gguf_tensor_info(os.fsencode(path), name.encode(), ctypes.byref(t), _p(ne),
                                        ctypes.byref(off), ctypes.byref(nb))
    check(min(rc, 0))  # >= 0: the tensor count
    return t.value, tuple(int(v) for v in ne), off.value, nb.value


def gguf_tensor_count(path):
    n = lib().tie_hip_gguf_tensor_info(os.fsencode(path), None, None, None, None, None)
    check(min(n, 0))
    return n


def gguf_inspect(path):
    """tie_hip_gguf_inspect: the MoE shape of a GGUF file (no GPU needed)."""
    info = ModelInfo()
    check(lib().tie_hip_gguf_inspect(os.fsencode(path), ctypes.byref(info)))
    return info


class _LayerRef:
    """A layer owned by a Model (forward/forward_residual of Layer, no close)."""

    def __init__(self, handle):
        self.handle = handle

    forward = lambda self, *a, **kw: Layer.forward(self, *a, **kw)  # noqa: E731
    forward_residual = lambda self, *a, **kw: Layer.forward_residual(self, *a, **kw)  # noqa: E731


class Model:
    """tie_hip_gguf_load: every MoE layer of a GGUF file on the device."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().tie_hip_gguf_load(os.fsencode(path), ctypes.byref(h)))
        self.handle = h
        self.info = ModelInfo()
        lib().tie_hip_model_info_get(h, ctypes.byref(self.info))

    def layer(self, n):
        h = lib().tie_hip_model_layer(self.handle, n)
        return _LayerRef(ctypes.c_void_p(h)) if h else None

    def ffn_norm(self, n):
        """Device pointer (int) of layer n's ffn_norm, or None."""
        return lib().tie_hip_model_ffn_norm(self.handle, n)

    def close(self):
        if self.handle:
            lib().tie_hip_model_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Matrix:
    """A device-resident dense weight matrix (tie_hip_matrix_create):
    GGUF layout [rows][in_dim] of type F32, Q4_K, Q6_K or BF16."""

    def __init__(self, w, wtype, rows, in_dim, on_device=False):
        self.rows, self.in_dim = rows, in_dim
        h = ctypes.c_void_p()
        check(lib().tie_hip_matrix_create(_p(w), wtype, rows, in_dim, int(on_device), ctypes.byref(h)))
        self.handle = h

    def mat_mat(self, x_dev, T, out_dev, flags=PATH_AUTO, stream=None):
        """out[t][r] = W[r] . x[t] on device pointers (dispatch_mat_mat);
        PATH_AUTO takes the matrix cores above the exact threshold where the
        matrix allows them, PATH_EXACT always TIE's row kernels."""
        check(lib().tie_hip_mat_mat(self.handle, _p(x_dev), T, _p(out_dev), flags, stream))

    def close(self):
        if self.handle:
            lib().tie_hip_matrix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Layer:
    """A device-resident layer (tie_hip_layer_create).  Weight sources are
    host numpy arrays or device tensors (anything with data_ptr())."""

    def __init__(self, d, F, E, router, gate, up, down, gate_type, up_type, down_type, bias=None,
                 on_device=False, literal_bf16_stride=False, routing=ROUTE_SOFTMAX, probs_bias=None):
        self.d, self.F, self.E = d, F, E
        desc = LayerDesc(d, F, E, _p(router), F32, _p(gate), gate_type, _p(up), up_type, _p(down), down_type,
                         _p(bias), int(on_device), int(literal_bf16_stride), int(routing), _p(probs_bias))
        h = ctypes.c_void_p()
        check(lib().tie_hip_layer_create(ctypes.byref(desc), ctypes.byref(h)))
        self.handle = h

    @classmethod
    def from_synth(cls, s, literal_bf16_stride=False):
        return cls(s.d, s.F, s.E, s.router, s.gate, s.up, s.down, s.gate_type, s.up_type, s.down_type,
                   bias=s.bias, literal_bf16_stride=literal_bf16_stride,
                   routing=getattr(s, "routing", ROUTE_SOFTMAX), probs_bias=getattr(s, "probs_bias", None))

    def nbytes(self):
        return lib().tie_hip_layer_bytes(self.handle)

    def shifts(self):
        """(h_shift, y_shift): the matrix-core path's f16 scales of h and y."""
        h, y = ctypes.c_int(0), ctypes.c_int(0)
        check(lib().tie_hip_debug_layer_shifts(self.handle, ctypes.byref(h), ctypes.byref(y)))
        return h.value, y.value

    def forward(self, x_dev, T, k, out_dev, topk_idx_dev=None, topk_w_dev=None, flags=PATH_AUTO, stream=None):
        """Enqueue the block on device pointers (torch tensors or ints)."""
        check(lib().tie_hip_moe_forward(self.handle, _p(x_dev), T, k, _p(out_dev), _p(topk_idx_dev),
                                        _p(topk_w_dev), flags, stream))

    def forward_noalloc(self, x_dev, T, k, out_dev, topk_idx_dev=None, topk_w_dev=None, flags=PATH_AUTO,
                        stream=None):
        """tie_hip_moe_forward_noalloc: forward with the library's static
        scratch array (no allocation; small T only)."""
        check(lib().tie_hip_moe_forward_noalloc(self.handle, _p(x_dev), T, k, _p(out_dev), _p(topk_idx_dev),
                                                _p(topk_w_dev), flags, stream))

    def forward_residual(self, hidden_dev, ffn_norm_dev, eps, T, k, out_dev=None, topk_idx_dev=None,
                         topk_w_dev=None, flags=PATH_AUTO, stream=None):
        """out = hidden + block(rms_norm(hidden)) on device pointers (out
        defaults to hidden: the in-place update)."""
        check(lib().tie_hip_moe_forward_residual(self.handle, _p(hidden_dev), _p(ffn_norm_dev), eps, T, k,
                                                 _p(hidden_dev if out_dev is None else out_dev), _p(topk_idx_dev),
                                                 _p(topk_w_dev), flags, stream))

    def close(self):
        if self.handle:
            lib().tie_hip_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
