"""Seeded synthetic GGUF-layout tensors for the Qwen3-MoE FFN block.

Workload generator for tests and bench.py.  Byte layouts follow TIE's block
structs (gguf.h:100-113): Q4_K is 144 B per 256 weights (fp16 d, fp16 dmin,
12 packed 6-bit scale/min bytes, 128 nibble bytes); Q6_K is 210 B per 256
weights (128 B low nibbles, 64 B high 2-bit pairs, 16 int8 scales, fp16 d).
Stacked expert tensors are [E][rows][in] in GGUF order (ne = [in, rows, E]),
so expert e of a tensor with R rows starts at e * R * row_bytes.

Distributions (the workload configs of the MoE block):
  router  F32 ~ N(0, 0.02)
  Q4_K    uniform random bytes; d, dmin = fp16(|N(0, 0.01)|)
  Q6_K    uniform random ql/qh bytes; scales int8 uniform in [-32, 31];
          d = fp16(|N(0, 0.01)|)
  BF16    round-to-nearest-even bf16 of N(0, 0.02)
  x       F32 ~ N(0, 1)
"""
import hashlib

import numpy as np

F32, Q4_K, Q6_K, BF16 = 0, 12, 14, 30
TYPE_NAMES = {F32: "F32", Q4_K: "Q4_K", Q6_K: "Q6_K", BF16: "BF16"}
QK_K = 256
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}


def row_bytes(wtype, in_dim):
    if wtype == F32:
        return 4 * in_dim
    if wtype == BF16:
        return 2 * in_dim
    return (in_dim // QK_K) * BLOCK_BYTES[wtype]


def tensor_bytes(wtype, rows, in_dim, n_mat=1):
    return n_mat * rows * row_bytes(wtype, in_dim)


def _half_abs_normal(rng, n, scale):
    return np.abs(rng.normal(0.0, scale, size=n)).astype(np.float16)


def f32_to_bf16_bits(a):
    """Round-to-nearest-even bf16 bits of finite float32 values."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))  # no wrap for finite values
    return (r >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def q4k_blocks(rng, n_blocks):
    b = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    d = _half_abs_normal(rng, n_blocks, 0.01)
    dmin = _half_abs_normal(rng, n_blocks, 0.01)
    b[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    b[:, 2:4] = dmin.view(np.uint8).reshape(n_blocks, 2)
    return b


def q6k_blocks(rng, n_blocks):
    b = rng.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    sc = rng.integers(-32, 32, size=(n_blocks, 16), dtype=np.int8)
    b[:, 192:208] = sc.view(np.uint8)
    d = _half_abs_normal(rng, n_blocks, 0.01)
    b[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return b


def expert_tensor(rng, wtype, n_exp, rows, in_dim):
    """Stacked [n_exp][rows][in_dim] expert tensor as a flat uint8 array."""
    if wtype == Q4_K:
        return q4k_blocks(rng, n_exp * rows * (in_dim // QK_K)).reshape(-1)
    if wtype == Q6_K:
        return q6k_blocks(rng, n_exp * rows * (in_dim // QK_K)).reshape(-1)
    if wtype == BF16:
        # drawn in chunks: the same stream of normals as one draw, in less memory
        n = n_exp * rows * in_dim
        out = np.empty(n, np.uint16)
        step = 1 << 24
        for i in range(0, n, step):
            m = min(step, n - i)
            out[i:i + m] = f32_to_bf16_bits(rng.normal(0.0, 0.02, size=m).astype(np.float32))
        return out.view(np.uint8)
    raise ValueError("unsupported expert type %r" % (wtype,))


def zipf_bias(n_exp, s=1.2, c=1.0, seed=0):
    """Per-expert router-logit offset c * rank^-s over a seeded permutation of
    the experts (the load-imbalanced routing config)."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(n_exp) + 1
    return (c * ranks.astype(np.float64) ** (-s)).astype(np.float32)


class MoELayer:
    """One MoE FFN layer's weights in host memory, GGUF layout."""

    def __init__(self, d, F, E, gate, up, down, router, gu_type, down_type, bias=None, routing=0,
                 probs_bias=None):
        self.d, self.F, self.E = d, F, E
        self.gate, self.up, self.down, self.router = gate, up, down, router
        self.gate_type = self.up_type = gu_type
        self.down_type = down_type
        self.bias = bias
        # 0: softmax routing (Qwen3); 1: sigmoid routing with an optional
        # selection bias (LFM2's exp_probs_b_bias)
        self.routing = routing
        self.probs_bias = probs_bias

    def digest(self):
        h = hashlib.sha256()
        for a in (self.router, self.gate, self.up, self.down):
            h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
        return h.hexdigest()


def make_layer(seed, d, F, E, gu_type=Q4_K, down_type=Q6_K, zipf=None, routing=0, probs_bias=None):
    """probs_bias: None, or the standard deviation of a seeded N(0, s)
    selection bias for sigmoid routing (LFM2's exp_probs_b_bias)."""
    rng = np.random.default_rng(seed)
    router = rng.normal(0.0, 0.02, size=(E, d)).astype(np.float32)
    gate = expert_tensor(rng, gu_type, E, F, d)
    up = expert_tensor(rng, gu_type, E, F, d)
    down = expert_tensor(rng, down_type, E, d, F)
    bias = zipf_bias(E, s=zipf, seed=seed + 7) if zipf else None
    pb = None
    if probs_bias:
        pb = np.random.default_rng(seed + 11).normal(0.0, probs_bias, size=E).astype(np.float32)
    return MoELayer(d, F, E, gate, up, down, router, gu_type, down_type, bias, routing, pb)


def make_norm_weight(seed, d):
    """RMSNorm weight (ffn_norm) ~ N(1, 0.1), seeded."""
    rng = np.random.default_rng(seed + 2000003)
    return rng.normal(1.0, 0.1, size=d).astype(np.float32)


def make_input(seed, T, d):
    rng = np.random.default_rng(seed + 1000003)
    return rng.normal(0.0, 1.0, size=(T, d)).astype(np.float32)


# The workload configs of the MoE block benchmark (30B-A3B / 235B-A22B shapes;
# lfm2_*: LFM2-8B-A1B-shaped blocks with sigmoid routing and a selection bias;
# *_ffn: the FFN half of the layer, RMSNorm before and the residual add after).
CONFIGS = {
    "30b_t1": dict(d=2048, F=768, E=128, k=8, T=1, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1234),
    "30b_t2": dict(d=2048, F=768, E=128, k=8, T=2, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1242),
    "30b_t4": dict(d=2048, F=768, E=128, k=8, T=4, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1244),
    "30b_t8": dict(d=2048, F=768, E=128, k=8, T=8, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1240),
    "30b_t12": dict(d=2048, F=768, E=128, k=8, T=12, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1280),
    "30b_t14": dict(d=2048, F=768, E=128, k=8, T=14, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1281),
    "30b_t16": dict(d=2048, F=768, E=128, k=8, T=16, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1252),
    "30b_t20": dict(d=2048, F=768, E=128, k=8, T=20, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1257),
    "30b_t22": dict(d=2048, F=768, E=128, k=8, T=22, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1259),
    "30b_t24": dict(d=2048, F=768, E=128, k=8, T=24, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1253),
    "30b_t32": dict(d=2048, F=768, E=128, k=8, T=32, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1235),
    "30b_t64": dict(d=2048, F=768, E=128, k=8, T=64, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1243),
    "30b_t128": dict(d=2048, F=768, E=128, k=8, T=128, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1245),
    "30b_t256": dict(d=2048, F=768, E=128, k=8, T=256, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1246),
    "30b_t192": dict(d=2048, F=768, E=128, k=8, T=192, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1282),
    "30b_t256": dict(d=2048, F=768, E=128, k=8, T=256, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1283),
    "30b_t384": dict(d=2048, F=768, E=128, k=8, T=384, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1284),
    "30b_t512": dict(d=2048, F=768, E=128, k=8, T=512, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1247),
    "30b_t1024": dict(d=2048, F=768, E=128, k=8, T=1024, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1248),
    "30b_t32_ffn": dict(d=2048, F=768, E=128, k=8, T=32, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1235,
                        residual=True),
    "30b_t2048": dict(d=2048, F=768, E=128, k=8, T=2048, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1236),
    "30b_bf16_zipf_t512": dict(d=2048, F=768, E=128, k=8, T=512, gu_type=BF16, down_type=BF16, zipf=1.2,
                               seed=1237),
    "235b_t1": dict(d=4096, F=1536, E=128, k=8, T=1, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1238),
    "lfm2_t1": dict(d=2048, F=1792, E=32, k=4, T=1, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1250,
                    routing=1, probs_bias=0.05),
    "lfm2_t32": dict(d=2048, F=1792, E=32, k=4, T=32, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1251,
                     routing=1, probs_bias=0.05),
    # dense matrices (dispatch_mat_mat): a q_proj-shaped Q4_K matrix and a
    # Q6_K LM head (151936 x 2048) of the 30B model
    "dense_q4k_t1": dict(kind="dense", rows=4096, **{"in": 2048}, wtype=Q4_K, T=1, seed=1270),
    "dense_q4k_t32": dict(kind="dense", rows=4096, **{"in": 2048}, wtype=Q4_K, T=32, seed=1271),
    "lmhead_q6k_t1": dict(kind="dense", rows=151936, **{"in": 2048}, wtype=Q6_K, T=1, seed=1272),
    "dense_q4k_t32_mfma": dict(kind="dense", rows=4096, **{"in": 2048}, wtype=Q4_K, T=32, seed=1271, path="mfma"),
    "dense_q4k_t512": dict(kind="dense", rows=4096, **{"in": 2048}, wtype=Q4_K, T=512, seed=1273, path="mfma"),
    "dense_q6k_t2048": dict(kind="dense", rows=4096, **{"in": 4096}, wtype=Q6_K, T=2048, seed=1274, path="mfma"),
    "235b_t1024": dict(d=4096, F=1536, E=128, k=8, T=1024, gu_type=Q4_K, down_type=Q6_K, zipf=None, seed=1239),
}
