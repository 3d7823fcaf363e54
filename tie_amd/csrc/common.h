// common.h -- shared definitions of the gfx950 MoE block kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/tie_hip.h"

namespace tie {

constexpr int QK = 256;          // weights per K-quant super-block
constexpr int Q4K_BYTES = 144;   // block_q4_k (gguf.h:108-113)
constexpr int Q6K_BYTES = 210;   // block_q6_k (gguf.h:101-106)
constexpr int PANEL_ROWS = 64;   // rows per weight panel = one wave64, one row per lane
constexpr int Q4K_CHUNKS = 9;    // 144 B = 9 x 16 B
constexpr int Q6K_CHUNKS = 13;   // ql 8 + qh 4 + scales 1 chunks of 16 B; d in a 128 B plane
constexpr size_t Q4K_PANEL = (size_t)PANEL_ROWS * Q4K_BYTES; // 9216
constexpr size_t Q6K_PANEL = (size_t)PANEL_ROWS * Q6K_BYTES; // 13440
constexpr int MAX_K = 32;
constexpr int MAX_E = 1024;
constexpr int SILU_N = TIE_SILU_TABLE_SIZE;
// MFMA work tiles: pair rows of one expert per tile at most, gate/up and
// down (each kernel has its own tile list; MFMA_MT is the larger)
#ifndef TIE_MFMA_MT_GU
#define TIE_MFMA_MT_GU 160
#endif
#ifndef TIE_MFMA_MT_DN
#define TIE_MFMA_MT_DN 128
#endif
constexpr int MFMA_MT_GU = TIE_MFMA_MT_GU;
constexpr int MFMA_MT_DN = TIE_MFMA_MT_DN;
constexpr int MFMA_MT = MFMA_MT_GU > MFMA_MT_DN ? MFMA_MT_GU : MFMA_MT_DN;
// gate/up tiles of the small-tile kernel (quantised weights, few pairs per
// expert: more waves per SIMD), used up to TIE_MFMA_SMALL_AVG pairs per expert
constexpr int MFMA_MT_GU_SMALL = 64;
// gate/up and down tiles of the BF16-weight kernels: short enough for two
// waves per SIMD with the weights prefetched into registers (30B BF16 Zipf
// T=512: gate/up 233 -> 213 us, down 127 -> 112 us against 160 / 128-row
// tiles at one wave per SIMD)
#ifndef TIE_MFMA_MT_GU_BF16
#define TIE_MFMA_MT_GU_BF16 96
#endif
constexpr int MFMA_MT_GU_BF16 = TIE_MFMA_MT_GU_BF16;
#ifndef TIE_MFMA_MT_DN_BF16
#define TIE_MFMA_MT_DN_BF16 96
#endif
constexpr int MFMA_MT_DN_BF16 = TIE_MFMA_MT_DN_BF16;
#ifndef TIE_MFMA_SMALL_AVG
#define TIE_MFMA_SMALL_AVG 32
#endif
// gate/up and down tiles of the tiny-tile kernels (32 rows; the LDS left
// over holds more weight stages in flight), used up to TIE_MFMA_TINY_AVG
// pairs per expert on average (16: 30B T=192 and T=256 3.6-4.9% faster
// than with 8, T=384 and T=512 slower with 24 or 32)
constexpr int MFMA_MT_TINY = 32;
// Up to this many tokens (an expert then has at most this many pairs: one
// 32-row tile), the 32-row-tile kernels run one work item per (expert,
// column slab) and h is laid out by expert ([E][MFMA_DIRECT_T][F]), so a
// workgroup finds its tile without a scan of the counts
constexpr int MFMA_DIRECT_T = 32;
#ifndef TIE_MFMA_TINY_AVG
#define TIE_MFMA_TINY_AVG 16
#endif

// Device layout of one stacked expert tensor [E][rows][in].
//
// Q4_K / Q6_K: "panels".  Rows are grouped 64 at a time (one per lane of a
// wave64); panel (e, rt, b) holds block column b of rows rt*64 .. rt*64+63
// of expert e.  Inside a panel, 16-byte chunk c of the block of lane i
// sits at c*1024 + i*16, so a wave reads each chunk of its 64 blocks with
// one fully coalesced 1 KiB global_load_dwordx4.  Q6_K's 210-byte blocks
// are split into ql (8 chunks), qh (4), scales (1) and a trailing plane of
// 64 fp16 d values, so the panel is exactly 64*210 bytes: no padding, no
// extra HBM traffic.  The panel is also the (64 x 256) weight tile the
// grouped GEMM dequantises into LDS.
//
// BF16: GGUF row-major [E][rows][in], unchanged.
struct ExpertTensor {
	const uint8_t *data = nullptr;
	int type = 0;
	int rows = 0, in = 0;   // per expert
	int nb = 0;             // in / 256 (quantised types)
	int rt = 0;             // rows / 64
	size_t expert_bytes = 0;
};

__host__ __device__ inline size_t panel_bytes(int type)
{
	return type == TIE_GGML_Q4_K ? Q4K_PANEL : Q6K_PANEL;
}

struct Layer {
	int d = 0, F = 0, E = 0;
	const float *router = nullptr; // [E][d]
	const float *routerT = nullptr; // [d][E] (the tiled router kernel's layout)
	const float *bias = nullptr;   // [E] or null, added to the logits
	int routing = 0;               // ROUTE_SOFTMAX (Qwen3) or ROUTE_SIGMOID (LFM2)
	const float *pbias = nullptr;  // [E] or null: LFM2 selection bias (exp_probs_b_bias)
	ExpertTensor gate, up, down;
	int h_shift = 0;               // MFMA path: h is stored as f16(h * 2^-h_shift)
	int y_shift = 0;               // MFMA path, quantised down: y is stored as f16(y * 2^-y_shift)
	void *alloc = nullptr;         // one device allocation holding everything
	size_t bytes = 0;
};

// Per-forward scratch (grown on demand, one per device).
struct Workspace {
	int32_t *topk_idx = nullptr;  // [T][k]
	float *topk_w = nullptr;      // [T][k]
	int32_t *offsets = nullptr;   // [E+1]    start of each expert's pair list
	int32_t *pairs = nullptr;     // [T*k]    pair ids t*k+j grouped by expert
	int32_t *active = nullptr;    // [E+1]    active experts; active[E] = count
	float *logits = nullptr;      // [T][E]   router logits
	float *h = nullptr;           // [2][T*k][F] gate and up row sums (exact path)
	uint16_t *hb = nullptr;       // [T*k][F] SwiGLU activations (bf16 hi/lo, MFMA path)
	uint16_t *hd = nullptr;       // [E][MFMA_DIRECT_T][F] h by expert (decode-sized MFMA batches; null: none)
	float *y = nullptr;           // [T*k][d] expert outputs
	float *normed = nullptr;      // [T][d]   RMSNorm of the hidden state (residual forward)
	uint16_t *hlo = nullptr;      // [T*k][F] SwiGLU activations, bf16 remainder (MFMA path, BF16 weights)
	uint16_t *xb = nullptr;       // [T][d]   x as bf16 (MFMA path)
	uint16_t *xlo = nullptr;      // [T][d]   x - bf16(x) as bf16 (MFMA path, BF16 weights)
	uint16_t *xsum = nullptr;     // [T][2][d/32] sums of f16(x) over each 32-K sub-block as f16 high and
	                              //          remainder parts (MFMA path, Q4_K 32-row gate/up tiles)
	int32_t *bucket_cnt = nullptr; // [E]   MFMA path: pairs per expert
	uint8_t *sel = nullptr;       // [E][T4(T)] MFMA path: slot + 1 that chose the expert (0: none)
	int32_t *bucket = nullptr;    // [E][T4(T)] MFMA path: each expert's pair ids in token order
	int32_t *tok_flag = nullptr;  // [T]      f16 path: token's activations left the f16 range
	int32_t *fix_list = nullptr;  // [T]      flagged tokens (recomputed exactly after the forward)
	int32_t *fix_count = nullptr; // [1]
	unsigned long long *one_lg = nullptr; // [ONE_LG_COPIES][E, 4 KiB rows]  one-launch decode: {seq, logit} words
	unsigned long long *one_h = nullptr; // [ONE_H_COPIES][MAX_K * F, 4 KiB rows] one-launch decode: {seq, h} words
	uint32_t one_seq = 0;         // one-launch decode: sequence number of the last call
	int32_t *one_status = nullptr; // [1] one-launch decode: 1 when a wait gave up (outputs NaN)
	size_t cap_pairs = 0, cap_F = 0, cap_d = 0, cap_E = 0;
	void *alloc = nullptr;
};

// ---------------------------------------------------------------- launchers
// T rounded up to a multiple of 4 (the row stride of the MFMA path's
// per-expert selection bytes and pair lists)
inline int T4(int T)
{
	return (T + 3) & ~3;
}
// words the router logits kernel clears before the kernels that follow
// accumulate into them
struct ZeroArgs {
	int32_t *p = nullptr, *p2 = nullptr;
	int n = 0, n2 = 0;
	int32_t *one = nullptr;
};
// The matrix-core path's f16 A operand of x (gate/up; K order 0,2,1,3,4,6,5,7
// inside each group of 8) and the token's range flag (1: a value not finite
// or not below 65504 in magnitude), written by the tiled logits kernel from
// the x rows it stages anyway (router_converts_x); the routing kernel then
// only lists the flagged tokens.
struct XConvArgs {
	uint16_t *xa = nullptr;
	int32_t *flag = nullptr;
};
bool router_converts_x(const Layer &L, int T);
hipError_t launch_router_logits(const Layer &L, const float *x, int T, float *logits, hipStream_t s,
				ZeroArgs z = ZeroArgs(), XConvArgs xc = XConvArgs());
// the matrix-core path's routing appends its pairs to the per-expert lists
// (atomics on the counts) up to this many tokens; above, selection bytes
// and bucket_plan (contended atomics: T=2048 35 us against 10 us)
#ifndef TIE_ROUTE_APPEND_MAX_T
#define TIE_ROUTE_APPEND_MAX_T 256
#endif
constexpr int ROUTE_APPEND_MAX_T = TIE_ROUTE_APPEND_MAX_T;
inline bool route_appends(int T)
{
	return T <= ROUTE_APPEND_MAX_T;
}
// The matrix-core path's quantised down stores y as f16 scaled by the
// layer's 2^-y_shift (1) or as fp32 (0): f16 halves the bytes the down
// kernel writes and the combine reads, and adds 2^-12 relative rounding
// per element (about 2e-4 relative L2 at the block's output)
#ifndef TIE_MFMA_Y16
#define TIE_MFMA_Y16 1
#endif
// the matrix-core path's selection, grouping into per-expert buckets and
// A-operand conversion (mfma.hip)
// converted: the logits kernel wrote the f16 A operand and the range flags
// (XConvArgs); the routing then only lists the flagged tokens
hipError_t launch_route_bucket(const Layer &L, const float *x, int T, int k, Workspace &ws, hipStream_t s,
			       bool converted);
hipError_t launch_bucket_plan(const Layer &L, int T, int k, Workspace &ws, hipStream_t s);
hipError_t launch_router_select(const Layer &L, int T, int k, const float *logits, int32_t *topk_idx, float *topk_w,
				hipStream_t s);
hipError_t launch_router(const Layer &L, const float *x, int T, int k, float *logits, int32_t *topk_idx,
			 float *topk_w, hipStream_t s);
hipError_t launch_router_transpose(const Layer &L, hipStream_t s);
hipError_t launch_dispatch(const Layer &L, int T, int k, const int32_t *topk_idx, Workspace &ws, hipStream_t s);
hipError_t launch_route_group(const Layer &L, int T, int k, const float *logits, Workspace &ws, hipStream_t s);
hipError_t launch_exact_block(const Layer &L, const float *x, int T, int k, const float *silu, Workspace &ws,
			      float *out, hipStream_t s, const float *res = nullptr);
hipError_t launch_mfma_experts(const Layer &L, const float *x, int T, int k, const float *silu, Workspace &ws,
			       hipStream_t s);
// True when the matrix-core path of this layer takes f16 operands, whose
// range the forward guards (tokens outside it are recomputed exactly).
bool mfma_f16_operands(const Layer &L);
// The block for listed tokens in TIE's exact arithmetic (decode.hip): list
// == null runs token 0 of a one-token call (routed from its logits when
// inline_route, E <= 128); otherwise the *count tokens of list, with their
// selection already in topk_idx / topk_w.  h: [entries][k][F] scratch.
bool decode_supported(const Layer &L, int k);
// The f16 path's listed tokens recomputed exactly, a workgroup per token,
// in one launch (recompute_kernel); count on the device, T bounds it.
bool recompute_supported(const Layer &L, int k);
hipError_t launch_recompute(const Layer &L, const float *x, int k, const float *silu, const int32_t *topk_idx,
			    const float *topk_w, float *out, const float *res, const int32_t *list,
			    const int32_t *count, int T, hipStream_t s);
// The matrix-core path's combine (f16 y; tokens with skip[t] set left
// alone) and the exact recomputation of the listed tokens in one launch,
// when combine_fix_preferred
bool combine_fix_preferred(const Layer &L);
hipError_t launch_combine_fix(const Layer &L, const float *x, int k, const float *silu, const int32_t *topk_idx,
			      const float *topk_w, const void *y, bool y16, int y_shift, float *out, const float *res,
			      const int32_t *skip, const int32_t *list, const int32_t *count, int T, hipStream_t s);

hipError_t launch_decode(const Layer &L, const float *x, int k, const float *silu, const float *logits,
			 int32_t *topk_idx, float *topk_w, float *h, float *out, const float *res, const int32_t *list,
			 const int32_t *count, int max_entries, bool inline_route, bool fixup, hipStream_t s);
// T = 1 in one launch (router, gate/up and down + combine workgroups that
// hand the logits and h over as sequence-stamped words in lg / hw; E <= 128)
bool decode_one_supported(const Layer &L, int k);
hipError_t launch_decode_one(const Layer &L, const float *x, int k, const float *silu, int32_t *topk_idx,
			     float *topk_w, float *out, const float *res, unsigned long long *lg, size_t lg_copy,
			     unsigned long long *hw, size_t hw_copy, uint32_t seq, uint32_t wseq, int spin, int32_t *status,
			     hipStream_t s);
// polls before a wait of the one-launch decode gives up (each poll sleeps
// about 64 cycles: tens of milliseconds in all)
constexpr int ONE_SPIN_MAX = 1 << 18;
// The one-launch decode publishes the logits and h in several copies (4 KiB
// apart, so in different memory channels), each polled by a share of the
// reader workgroups: all readers polling one copy queue on its few lines.
#ifndef TIE_ONE_LG_COPIES
#define TIE_ONE_LG_COPIES 8
#endif
#ifndef TIE_ONE_H_COPIES
#define TIE_ONE_H_COPIES 1
#endif
constexpr int ONE_LG_COPIES = TIE_ONE_LG_COPIES, ONE_H_COPIES = TIE_ONE_H_COPIES;
// words between copies of n words
constexpr size_t one_copy_words(size_t n)
{
	return (n * 8 + 4095) / 4096 * 512;
}
struct Layer;
int mfma_gu_rows(const Layer &L, int npairs); // rows per gate/up tile (the tile list's and the kernel's)
int mfma_dn_rows(const Layer &L, int npairs); // rows per down tile
// Dense F32-input matrix product through the expert GEMV kernels: out[t][r]
// = W[r] . x[t] (W one "expert": rows, in, panel layout); dense_groups(T)
// token groups (the workspace needs that many experts and T pairs)
hipError_t launch_dense(const ExpertTensor &W, const float *x, int T, float *out, Workspace &ws, hipStream_t s);
// The same for a few tokens (T <= 4, Q4_K / Q6_K): a lane per (row, block),
// the block loaded once for all tokens (decode.hip); needs no workspace
bool dense_rows_supported(const ExpertTensor &W, int T);
hipError_t launch_dense_rows(const ExpertTensor &W, const float *x, int T, float *out, hipStream_t s);
bool dense_stream_supported(const ExpertTensor &W, int T);
hipError_t launch_dense_stream(const ExpertTensor &W, const float *x, float *out, hipStream_t s);
// TIE's exact rows of the tokens with flag[t] set (decode.hip)
hipError_t launch_dense_fix(const ExpertTensor &W, const float *x, int T, float *out, const int32_t *flag,
			    hipStream_t s);
// Dense Q4_K / Q6_K matrix product on the f16 matrix cores (mfma.hip): rows
// a multiple of 256; tokens whose x leaves the f16 range computed exactly
bool mfma_dense_supported(const ExpertTensor &W, int T);
hipError_t launch_mfma_dense(const ExpertTensor &W, const float *x, int T, float *out, Workspace &ws, hipStream_t s);
int dense_groups(int T);
// res (optional): out = res + combine (the residual add after the block)
// y16: y holds f16(y 2^-y_shift) (the matrix-core path's quantised down)
hipError_t launch_combine(int T, int d, int k, const float *topk_w, const int32_t *topk_idx, const float *y,
			  float *out, hipStream_t s, const float *res = nullptr, const int32_t *skip = nullptr,
			  bool y16 = false, int y_shift = 0);
// TIE's RMSNorm of each row of x into out; tab/nbits: the host RSQRTSS table
hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int T, int d, float *out, const uint32_t *tab,
			  int nbits, hipStream_t s);
hipError_t launch_repack(const ExpertTensor &dst, const uint8_t *src, int E, int literal_bf16_stride, hipStream_t s);

// Raise a kernel's dynamic-LDS limit to at least `bytes` (remembered per
// kernel: the attribute call runs only when a launch needs more)
hipError_t ensure_lds_limit(const void *fn, size_t bytes);

// Per-kernel timing (tie_hip_profile_enable): prof_begin / prof_end bracket
// a named section of launches; every kernel launched through tie_launch
// inside a section carries a start and a stop event bound to its own
// dispatch (hipExtLaunchKernel), so a section's time is the sum of its
// kernels' execution times, without the gaps that separate event records
// between launches would add.  No-ops while profiling is off.
void prof_begin(const char *name, hipStream_t s);
void prof_end(hipStream_t s);
// the event pair of the next launch in an open section (false: none)
bool prof_kernel_events(hipEvent_t *start, hipEvent_t *stop);

template <typename K, typename... A>
inline void tie_launch(K kern, dim3 grid, dim3 block, size_t lds, hipStream_t s, A... args)
{
	hipEvent_t e0, e1;
	if (prof_kernel_events(&e0, &e1))
		hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)lds, s, e0, e1, 0u, args...);
	else
		hipLaunchKernelGGL(kern, grid, block, lds, s, args...);
}

// ---------------------------------------------------------------- device helpers
#if defined(__HIPCC__)
// Copy n4 float4s from global memory with every thread of the workgroup,
// dst(q, v) storing element q (to LDS): each thread issues a batch of BATCH
// loads before the first store, so a copy of up to BATCH * blockDim.x
// elements costs one memory round trip instead of one per element it holds.
template <int BATCH, typename DST>
__device__ __forceinline__ void copy_in(const float4 *__restrict__ src, int n4, DST dst)
{
	for (int base = threadIdx.x; base < n4; base += BATCH * (int)blockDim.x) {
		float4 v[BATCH];
#pragma unroll
		for (int i = 0; i < BATCH; i++) {
			const int q = base + i * (int)blockDim.x;
			v[i] = src[q < n4 ? q : n4 - 1];
		}
#pragma unroll
		for (int i = 0; i < BATCH; i++) {
			const int q = base + i * (int)blockDim.x;
			if (q < n4)
				dst(q, v[i]);
		}
	}
}

// The 8-lane horizontal sum of an AVX2 accumulator (lo+hi, hadd, hadd).
__device__ __forceinline__ float hsum8(const float v[8])
{
	float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
	return (s0 + s1) + (s2 + s3);
}

// IEEE binary16 -> binary32, exact, in integer arithmetic (independent of
// the denormal mode).
__device__ __forceinline__ float half_bits_to_float(uint32_t h)
{
	uint32_t sign = (h & 0x8000u) << 16;
	uint32_t e = (h >> 10) & 0x1f;
	uint32_t m = h & 0x3ff;
	uint32_t bits;
	if (e == 0x1f) {
		bits = sign | 0x7f800000u | (m << 13);
	} else if (e != 0) {
		bits = sign | ((e + 112u) << 23) | (m << 13);
	} else if (m != 0) {
		// value m * 2^-24 with the leading one at bit p
		int p = 31 - __builtin_clz(m);
		bits = sign | ((uint32_t)(p + 103) << 23) | ((m << (23 - p)) & 0x7fffffu);
	} else {
		bits = sign;
	}
	return __uint_as_float(bits);
}

// Q6_K codes q = ql nibble | (qh 2-bit field << 4) of four weights, as the
// int8 bytes of q - 32 (exact: -32..31): the two high bits h select the
// signed top nibble (h - 2) << 4 from a byte table with one v_perm_b32, the
// nibble is or-ed in below it.  `hsh` is the field's shift in H (0, 2, 4,
// 6), `lsh` the nibble's in L (0, 4).  Each byte converts to float in one
// instruction (sbyte_f).
__device__ __forceinline__ uint32_t q6_codes(uint32_t L, int lsh, uint32_t H, int hsh)
{
	const uint32_t top = __builtin_amdgcn_perm(0u, 0x1000f0e0u, (H >> hsh) & 0x03030303u);
	return top | ((L >> lsh) & 0x0f0f0f0fu);
}

// signed byte i of w as a float
__device__ __forceinline__ float sbyte_f(uint32_t w, int i)
{
	return (float)(int8_t)((w >> (8 * i)) & 0xffu);
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b)
{
	return __uint_as_float(b << 16);
}

// TIE's table SiLU x gate (swiglu_activation_f32_f32_avx2,
// math_avx2.c:908-950): pos = ((x + 10) * 8191) * 0.05f, round half to even
// with CVTPS2DQ's INT_MIN for NaN / out-of-range, clamp to [0, 8190],
// interpolate with one FMA; then multiply by up.
__device__ __forceinline__ float tie_swiglu(float g, float u, const float *__restrict__ tab)
{
	float pos = ((g + 10.0f) * 8191.0f) * 0.05f;
	int idx;
	if (pos >= -2147483648.0f && pos < 2147483648.0f)
		idx = (int)__builtin_rintf(pos);
	else
		idx = (int)0x80000000;
	idx = idx < 0 ? 0 : idx;
	idx = idx > SILU_N - 2 ? SILU_N - 2 : idx;
	float frac = pos - (float)idx;
	float y1 = tab[idx], y2 = tab[idx + 1];
	float s = __builtin_fmaf(frac, y2 - y1, y1);
	return s * u;
}
// One token's combine over 8 columns (c8: 8-column group) of the expert
// outputs: out[t][c] = [res[t][c] +] sum_j fma(g_j, y[t*k+j][c], .) in slot
// order (model_qwen3.c:459-467, then the residual add of
// apply_residual_f32_f32_avx2, math_avx2.c:731-751).  y is fp32, or (Y16)
// f16 values scaled by 2^-y_shift, whose scale ysc = 2^y_shift is folded
// into g (a power of two: exact).  Slots of 8 loaded before their FMAs: one
// memory wait per 8 slots.
template <bool Y16>
__device__ __forceinline__ void combine8_cols(int t, int c8, int d, int k, const float *__restrict__ topk_w,
					      const int32_t *__restrict__ topk_idx, const void *__restrict__ yv, float ysc,
					      const float *res, float *out)
{
	float acc[8];
#pragma unroll
	for (int i = 0; i < 8; i++)
		acc[i] = 0.0f;
	constexpr int CG = 8;
	for (int j0 = 0; j0 < k; j0 += CG) {
		float4 v[CG][Y16 ? 1 : 2];
		float g[CG];
#pragma unroll
		for (int q = 0; q < CG; q++) {
			const int j = j0 + q;
			const bool on = j < k && topk_idx[t * k + (j < k ? j : 0)] >= 0;
			g[q] = on ? (Y16 ? topk_w[t * k + j] * ysc : topk_w[t * k + j]) : 0.0f;
			// every slot's row is loaded (its address does not wait for
			// topk_idx); a slot without an expert adds nothing
			const size_t row = (size_t)t * k + (j < k ? j : j0);
			if constexpr (Y16) {
				v[q][0] = reinterpret_cast<const float4 *>(reinterpret_cast<const uint16_t *>(yv) + row * d)[c8];
			} else {
				const float4 *yr = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(yv) + row * d) + 2 * c8;
				v[q][0] = yr[0];
				v[q][1] = yr[1];
			}
		}
#pragma unroll
		for (int q = 0; q < CG; q++) {
			const int j = j0 + q;
			if (j < k && topk_idx[t * k + j] >= 0) {
				float y[8];
				if constexpr (Y16) {
					typedef _Float16 h8 __attribute__((ext_vector_type(8)));
					const h8 hv = __builtin_bit_cast(h8, v[q][0]);
#pragma unroll
					for (int i = 0; i < 8; i++)
						y[i] = (float)hv[i];
				} else {
					const float4 a = v[q][0], b = v[q][1];
					y[0] = a.x, y[1] = a.y, y[2] = a.z, y[3] = a.w, y[4] = b.x, y[5] = b.y, y[6] = b.z, y[7] = b.w;
				}
#pragma unroll
				for (int i = 0; i < 8; i++)
					acc[i] = __builtin_fmaf(g[q], y[i], acc[i]);
			}
		}
	}
	float4 *o = reinterpret_cast<float4 *>(out + (size_t)t * d) + 2 * c8;
	float4 a = make_float4(acc[0], acc[1], acc[2], acc[3]), b = make_float4(acc[4], acc[5], acc[6], acc[7]);
	if (res) {
		const float4 *h = reinterpret_cast<const float4 *>(res + (size_t)t * d) + 2 * c8;
		const float4 h0 = h[0], h1 = h[1];
		a = make_float4(h0.x + a.x, h0.y + a.y, h0.z + a.z, h0.w + a.w);
		b = make_float4(h1.x + b.x, h1.y + b.y, h1.z + b.z, h1.w + b.w);
	}
	o[0] = a;
	o[1] = b;
}
#endif

} // namespace tie
