// exact.hip -- expert GEMVs that reproduce TIE's fp32 arithmetic bit for bit.
//
// Reference: process_expert_task (engine.c:916-964) runs, per selected
// expert, gate and up GEMVs (dispatch_mat_vec, engine.c:953-956), the table
// SwiGLU (engine.c:959) and the down GEMV (engine.c:962) with the AVX2 row
// kernels of math_avx2.c.  A quantised row is a serial fp32 sum over its
// super-blocks (math_avx2.c:753-787); each super-block dot is two 8-lane
// FMA accumulators reduced by hsum_f32_avx2 (Q4_K: :535-604, Q6_K:
// :411-495); a BF16 row is one 8-lane accumulator over the whole row
// (:188-226).  The kernels here keep every rounding step and the order of
// every sum, so their outputs equal TIE's exactly.
//
// Work decomposition ((token, slot) pairs grouped by expert):
//   exact_gu_kernel    one workgroup per (64-row panel, active expert,
//                      matrix); wave w owns super-block columns w, w+8, ..;
//                      lane i owns row i.  The lane's super-block is read
//                      once per group of up to 16 pairs with coalesced
//                      16-byte panel loads (in stages: the next 64-weight
//                      group's chunks in flight while one computes, so
//                      a third of the block is in registers) and
//                      dequantised once per 8 weights for up to 4 pairs
//                      at a time; the input row
//                      of each pair comes in through scalar loads (one
//                      address per wave), so it reaches the FMAs as SGPR
//                      operands.  Per-block dots meet in LDS and are added
//                      in block order.  Writes the gate and up row sums.
//                      For one token (E <= 128) every workgroup first
//                      selects the token's experts itself (top-k,
//                      softmax): no separate routing launch.
//   exact_down_kernel  one workgroup per (64-row panel of d, active
//                      expert).  The prologue forms h = silu_tab(gate) * up
//                      (swiglu_activation_f32_f32_avx2) for its pairs in
//                      LDS; the blocks then read h as LDS broadcasts.
//   BF16 weights       two threads per row, each owning four of the row's
//                      eight lane accumulators.
// No kernel waits on another workgroup: the only ordering is the launch
// order on the stream.
#include <cmath>
#include <map>
#include <tuple>
#include <type_traits>
#include <unordered_map>

#include "common.h"
#include "route.h"

namespace tie {

// Input rows of the gate/up GEMVs are read through the constant address
// space: every lane of a wave reads the same address, so the loads become
// scalar (s_load) and the values reach the FMAs as SGPR operands.
typedef const float __attribute__((address_space(4))) cfloat;
// h rows of the down GEMV are LDS broadcasts.
typedef const float __attribute__((address_space(3))) lfloat;

// The launders below are empty asm statements that make a value opaque to
// the compiler at one point of the instruction stream.  Volatile asm keeps
// its order, so a step fence (every accumulator of every pair made opaque)
// followed by the launders of a step's input pointers and quant words
// pins the step between the FMAs of the step before and after it: without
// that the scheduler hoists every input value and dequantised weight of a
// super-block to the top and runs out of registers.
__device__ __forceinline__ void launder(cfloat *&p)
{
	asm volatile("" : "+s"(p));
}
__device__ __forceinline__ void launder(lfloat *&p)
{
	asm volatile("" : "+v"(p));
}
template <int PC> __device__ __forceinline__ void step_fence(float (&a0)[PC][8], float (&a1)[PC][8])
{
#pragma unroll
	for (int p = 0; p < PC; p++) {
		asm volatile("" : "+v"(a0[p][0]), "+v"(a0[p][1]), "+v"(a0[p][2]), "+v"(a0[p][3]), "+v"(a0[p][4]),
				  "+v"(a0[p][5]), "+v"(a0[p][6]), "+v"(a0[p][7]));
		asm volatile("" : "+v"(a1[p][0]), "+v"(a1[p][1]), "+v"(a1[p][2]), "+v"(a1[p][3]), "+v"(a1[p][4]),
				  "+v"(a1[p][5]), "+v"(a1[p][6]), "+v"(a1[p][7]));
	}
}

// Tuning knobs (compile-time): the most pairs one dot product serves at a
// time, and an optional occupancy target for the quantised kernels.
// steps whose input values a block dot of 3 or more pairs requests at once
// (scalar loads; 2 lets the compiler merge them and issue them earlier)
#ifndef TIE_Q4K_XS4
#define TIE_Q4K_XS4 2
#endif
#ifndef TIE_Q6K_XS
#define TIE_Q6K_XS 2
#endif
#ifndef TIE_Q4K_XS1
#define TIE_Q4K_XS1 4
#endif
#ifndef TIE_Q4K_XS2
#define TIE_Q4K_XS2 2
#endif
#ifndef TIE_Q6K_XS1
#define TIE_Q6K_XS1 2
#endif
#ifndef TIE_EXACT_PCMAX
#define TIE_EXACT_PCMAX 4
#endif
#ifndef TIE_DOWN_PM2
#define TIE_DOWN_PM2 1
#endif
#ifdef TIE_EXACT_WPE
#define EXACT_OCC __attribute__((amdgpu_waves_per_eu(TIE_EXACT_WPE)))
#else
#define EXACT_OCC
#endif
#ifdef TIE_GU_WPE
#define GU_OCC __attribute__((amdgpu_waves_per_eu(TIE_GU_WPE)))
#else
#define GU_OCC
#endif

// waves per split gate/up workgroup (one matrix, one token); the fused
// gate/up and the down kernels take their wave count from the launch
#ifndef TIE_GU_WAVES
#define TIE_GU_WAVES 8
#endif
#ifndef TIE_GU_PG
#define TIE_GU_PG 8
#endif

constexpr int GU_WAVES = TIE_GU_WAVES;
constexpr int GU_THREADS = 64 * GU_WAVES;
constexpr int PG_MAX = 16;        // pairs per LDS group
constexpr int PART_FLOATS = 16384; // LDS budget of the per-block partial dots (64 KiB)
// Routing in the gate/up prologue up to this T (E <= 128).  Only one token:
// for T = 2..8 every workgroup repeating the selection and grouping of all
// tokens costs more (T = 8: 64 us of gate/up against 33 us plus a 9.5 us
// grouping launch) than the launch it saves.
constexpr int INLINE_T = 1;
constexpr int INLINE_E = 128;

// ------------------------------------------------------------------ blocks
__device__ __forceinline__ uint32_t word(const uint4 &v, int i)
{
	return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ float ubyte(uint32_t w, int i)
{
	return (float)((w >> (8 * i)) & 0xffu);
}

// dot_product_f32_q4k_avx2 (math_avx2.c:535-604) of the lane's block with
// PC input rows at once.  Each weight w = fma(q, d*sc, -(dmin*m)) is formed
// once and used by the PC pairs; every pair keeps its own 16 accumulators
// and sees exactly TIE's sequence of FMAs.  32 steps s = (g, o, h) of 8
// weights each; step s reads x[64g + 16o + 4h + i] and x[.. + 32], loaded
// for a super-step of XS steps at once (two runs of 4*XS floats per pair, in
// SGPRs), so one wait for scalar loads covers XS steps of FMAs.
//
// The block is read in stages instead of at once: the scale chunk and
// the two quant chunks of 64-weight group 0 first, then the chunks of group
// g + 1 while group g computes.  That keeps 12 of the block's 36 dwords in
// registers at a time (vector loads return in order, so the wait for group
// g leaves group g + 1 in flight).
// Panel chunks through a global-address-space pointer: after a launder the
// loads stay global loads (a generic pointer would make them flat loads,
// which also count as LDS/scalar operations, so every wait for the scalar
// input loads would also wait for the next group's chunks).
typedef const uint4 __attribute__((address_space(1))) guint4;
typedef const uint16_t __attribute__((address_space(1))) guint16;
__device__ __forceinline__ uint4 ld(guint4 *p)
{
	return *(const uint4 *)p;
}

struct Q4KStream {
	guint4 *p; // the lane's first chunk; chunk c at p[64 c]
};

__device__ __forceinline__ void load_block(const uint8_t *__restrict__ panel, int lane, Q4KStream &S)
{
	S.p = (guint4 *)reinterpret_cast<const uint4 *>(panel) + lane;
}

__device__ __forceinline__ void launder(guint4 *&p)
{
	asm volatile("" : "+v"(p));
}

// Sub-block scale and negated minimum of Q4_K sub-block j (get_scale_min_k4,
// math_scalar.c:91-100) from the 12 packed bytes s[0..2].
__device__ __forceinline__ void q4k_sub_scale(const uint32_t s[3], int j, float d, float dmin, float &D, float &nM)
{
	auto sb = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
	uint32_t sc, m;
	if (j < 4) {
		sc = sb(j) & 63u;
		m = sb(j + 4) & 63u;
	} else {
		sc = (sb(j + 4) & 15u) | ((sb(j - 4) >> 6) << 4);
		m = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
	}
	D = d * (float)sc;
	nM = -(dmin * (float)m);
}

template <int PC, typename XP>
__device__ __forceinline__ void block_dots(const Q4KStream &S, XP *const xs[PC], float out[PC])
{
	const uint4 c0 = ld(S.p);
	uint4 cur[2] = {ld(S.p + 64), ld(S.p + 128)};
	const float d = half_bits_to_float(c0.x & 0xffffu);
	const float dmin = half_bits_to_float(c0.x >> 16);
	const uint32_t s[3] = {c0.y, c0.z, c0.w};
	float a0[PC][8], a1[PC][8];
#pragma unroll
	for (int p = 0; p < PC; p++)
#pragma unroll
		for (int l = 0; l < 8; l++)
			a0[p][l] = a1[p][l] = 0.0f;
	constexpr int XS = PC == 1 ? TIE_Q4K_XS1 : PC == 2 ? TIE_Q4K_XS2 : TIE_Q4K_XS4;
	XP *xb[PC];
#pragma unroll
	for (int g = 0; g < 4; g++) {
		step_fence<PC>(a0, a1);
		uint4 nxt[2];
		if (g < 3) {
			guint4 *q = S.p + 64 * (3 + 2 * g);
			launder(q);
			nxt[0] = ld(q);
			nxt[1] = ld(q + 64);
			__builtin_amdgcn_sched_barrier(0);
		}
		float D1, M1, D2, M2;
		q4k_sub_scale(s, 2 * g, d, dmin, D1, M1);
		q4k_sub_scale(s, 2 * g + 1, d, dmin, D2, M2);
#pragma unroll
		for (int ss = 0; ss < 8; ss++) {
			const int st = 8 * g + ss, o = ss >> 2, h = ss & 3;
			step_fence<PC>(a0, a1);
			if (st % XS == 0) {
#pragma unroll
				for (int p = 0; p < PC; p++) {
					xb[p] = xs[p] + 64 * g + 16 * o + 4 * h;
					launder(xb[p]);
				}
			}
			uint32_t w = word(cur[o], h);
			asm volatile("" : "+v"(w));
			uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
			asm volatile("" : "+v"(lo), "+v"(hi));
			float wl[4], wh[4];
#pragma unroll
			for (int i = 0; i < 4; i++) {
				wl[i] = __builtin_fmaf(ubyte(lo, i), D1, M1);
				wh[i] = __builtin_fmaf(ubyte(hi, i), D2, M2);
			}
			const int xo = 4 * (st % XS);
#pragma unroll
			for (int p = 0; p < PC; p++) {
#pragma unroll
				for (int i = 0; i < 4; i++) {
					const int m = 4 * h + i;
					float &A = (m < 8) ? a0[p][m & 7] : a1[p][m & 7];
					A = __builtin_fmaf(xb[p][xo + i], wl[i], A);
					A = __builtin_fmaf(xb[p][xo + 32 + i], wh[i], A);
				}
			}
		}
		if (g < 3) {
			cur[0] = nxt[0];
			cur[1] = nxt[1];
		}
	}
#pragma unroll
	for (int p = 0; p < PC; p++) {
		float v[8];
#pragma unroll
		for (int l = 0; l < 8; l++)
			v[l] = a0[p][l] + a1[p][l];
		out[p] = hsum8(v);
	}
}

// dot_product_f32_q6k_avx2 (math_avx2.c:411-495) of the lane's block with
// PC input rows.  Panel chunks: 0-7 ql[0..127], 8-11 qh[0..63], 12 the
// int8 scales.  q - 32 is formed once per weight (q6_codes); per pair TIE's
// fma(d*sc, (q - 32) * x, acc) follows, the product rounded on its own.
// 16 steps s = (n, l, hw) of 16 weights each; step s reads x[128n + l +
// 4hw + i + {0, 32, 64, 96}].
//
// The block is read in stages: the scale chunk, d and the three quant
// chunks (ql low/high nibble sources and qh) of quarter (n, l >> 4) first,
// then those of the next quarter while one quarter computes.
struct Q6KStream {
	guint4 *p;    // the lane's first chunk; chunk c at p[64 c]
	guint16 *dp;  // the lane's d
};

__device__ __forceinline__ void load_block(const uint8_t *__restrict__ panel, int lane, Q6KStream &S)
{
	S.p = (guint4 *)reinterpret_cast<const uint4 *>(panel) + lane;
	S.dp = (guint16 *)reinterpret_cast<const uint16_t *>(panel + Q6K_CHUNKS * 1024) + lane;
}

template <int PC, typename XP>
__device__ __forceinline__ void block_dots(const Q6KStream &S, XP *const xs[PC], float out[PC])
{
	const uint4 sc4 = ld(S.p + 64 * 12);
	const float d = half_bits_to_float(*(const uint16_t *)S.dp);
	// quarter qt = (n, hl): chunks 4n + hl (ql, low nibbles), 4n + 2 + hl
	// (ql, high nibbles), 8 + 2n + hl (qh)
	auto quarter = [&](int qt, uint4 (&c)[3]) {
		const int n = qt >> 1, hl = qt & 1;
		guint4 *q = S.p + 64 * (4 * n + hl);
		launder(q);
		c[0] = ld(q);
		c[1] = ld(q + 128);
		c[2] = ld(q + 64 * (8 + 2 * n + hl) - 64 * (4 * n + hl));
	};
	uint4 cur[3];
	quarter(0, cur);
	float a0[PC][8], a1[PC][8];
#pragma unroll
	for (int p = 0; p < PC; p++)
#pragma unroll
		for (int l = 0; l < 8; l++)
			a0[p][l] = a1[p][l] = 0.0f;
	constexpr int XS = PC == 1 ? TIE_Q6K_XS1 : TIE_Q6K_XS;
	auto sc = [&](int j) { return (float)(int8_t)((word(sc4, j >> 2) >> (8 * (j & 3))) & 0xffu); };
	XP *xb[PC];
#pragma unroll
	for (int qt = 0; qt < 4; qt++) {
		step_fence<PC>(a0, a1);
		uint4 nxt[3];
		if (qt < 3) {
			quarter(qt + 1, nxt);
			__builtin_amdgcn_sched_barrier(0);
		}
#pragma unroll
		for (int ss = 0; ss < 4; ss++) {
			const int st = 4 * qt + ss;
			const int n = st >> 3, l = 8 * ((st >> 1) & 3), hw = st & 1;
			const int is = (l >= 16) ? 1 : 0;
			step_fence<PC>(a0, a1);
			if (st % XS == 0) {
#pragma unroll
				for (int p = 0; p < PC; p++) {
					xb[p] = xs[p] + 128 * n + l + 4 * hw;
					launder(xb[p]);
				}
			}
			const float W0 = d * sc(8 * n + is + 0);
			const float W1 = d * sc(8 * n + is + 2);
			const float W2 = d * sc(8 * n + is + 4);
			const float W3 = d * sc(8 * n + is + 6);
			const int dw = ((l & 8) >> 2) + hw;
			uint32_t L = word(cur[0], dw), L2 = word(cur[1], dw), H = word(cur[2], dw);
			asm volatile("" : "+v"(L), "+v"(L2), "+v"(H));
			// bytes of q - 32
			uint32_t q1 = q6_codes(L, 0, H, 0), q2 = q6_codes(L2, 0, H, 2);
			uint32_t q3 = q6_codes(L, 4, H, 4), q4 = q6_codes(L2, 4, H, 6);
			// two halves: words 1, 2 (accumulators a0, a1 via runs 0 and
			// 32), then words 3, 4 (runs 64 and 96); every accumulator keeps
			// TIE's order, and only eight converted weights are live
			const int xo = 4 * (st % XS);
#pragma unroll
			for (int half = 0; half < 2; half++) {
				uint32_t qa = half ? q3 : q1, qb = half ? q4 : q2;
				asm volatile("" : "+v"(qa), "+v"(qb));
				const float Wa = half ? W2 : W0, Wb = half ? W3 : W1;
				float fa[4], fb[4];
#pragma unroll
				for (int i = 0; i < 4; i++) {
					fa[i] = sbyte_f(qa, i);
					fb[i] = sbyte_f(qb, i);
				}
#pragma unroll
				for (int p = 0; p < PC; p++) {
#pragma unroll
					for (int i = 0; i < 4; i++) {
						const int m = 4 * hw + i;
						XP *xq = xb[p] + xo + i + 64 * half;
						a0[p][m] = __builtin_fmaf(Wa, fa[i] * xq[0], a0[p][m]);
						a1[p][m] = __builtin_fmaf(Wb, fb[i] * xq[32], a1[p][m]);
					}
				}
				if (half == 0)
					step_fence<PC>(a0, a1);
			}
		}
		if (qt < 3) {
#pragma unroll
			for (int i = 0; i < 3; i++)
				cur[i] = nxt[i];
		}
	}
#pragma unroll
	for (int p = 0; p < PC; p++) {
		float v[8];
#pragma unroll
		for (int l = 0; l < 8; l++)
			v[l] = a0[p][l] + a1[p][l];
		out[p] = hsum8(v);
	}
}

template <int TYPE> struct BlockOf;
template <> struct BlockOf<TIE_GGML_Q4_K> {
	using type = Q4KStream;
};
template <> struct BlockOf<TIE_GGML_Q6_K> {
	using type = Q6KStream;
};

// PC pairs of the group against the lane's block; part[(b*pg_cap + q) * 64 + lane]
template <int PC, typename Block, typename XP, typename XF>
__device__ __forceinline__ void pairs_chunk(const Block &blk, int q, XF xrow, float *part_b, int lane)
{
	XP *xs[PC];
#pragma unroll
	for (int p = 0; p < PC; p++)
		xs[p] = xrow(q + p);
	float out[PC];
	block_dots<PC>(blk, xs, out);
#pragma unroll
	for (int p = 0; p < PC; p++)
		part_b[(q + p) * 64 + lane] = out[p];
}

// All np pairs of a group against the lane's block: up to PM at a time, the remainder (1 .. PCMAX-1) in one chunk of its own size, so
// an expert with at most PCMAX pairs dequantises each weight once.
template <int PM, typename Block, typename XP, typename XF>
__device__ __forceinline__ void block_all_pairs(const Block &blk, int np, XF xrow, float *part_b, int lane)
{
	int q = 0;
	for (; q + PM <= np; q += PM)
		pairs_chunk<PM, Block, XP>(blk, q, xrow, part_b, lane);
	switch (np - q) {
	case 3:
		if constexpr (PM > 3)
			pairs_chunk<3, Block, XP>(blk, q, xrow, part_b, lane);
		break;
	case 2:
		if constexpr (PM > 2)
			pairs_chunk<2, Block, XP>(blk, q, xrow, part_b, lane);
		break;
	case 1:
		if constexpr (PM > 1)
			pairs_chunk<1, Block, XP>(blk, q, xrow, part_b, lane);
		break;
	default:
		break;
	}
}

// ------------------------------------------------------------ routing
struct ExactArgs {
	const uint8_t *w[2];  // gate/up (or down) tensor data, panel layout / BF16 row-major
	size_t expert_bytes[2];
	int rows, in, k, E, T;
	const float *x;       // [T][d] (gate/up)
	float *sums[2];       // [pairs][F] gate and up row sums (gate/up output, down input)
	float *y;             // [pairs][d] down output
	float *hbuf;          // [pairs][F] SwiGLU output (fused gate/up -> down)
	const float *silu;
	const float *logits;  // [T][E] (inline routing)
	int32_t *topk_idx;    // [T][k]
	float *topk_w;        // [T][k]
	int32_t *offsets, *pairs, *active; // grouping (global)
	int pg_cap;           // pairs per LDS group
	int inline_route;
	int single;           // T = 1 mode: slot j = pair j of expert topk_idx[j], no grouping
	int routing;          // ROUTE_SOFTMAX / ROUTE_SIGMOID (inline routing)
	const float *pbias;   // [E] selection bias of ROUTE_SIGMOID, or null
};

// Selection and grouping of all T <= INLINE_T tokens by one workgroup of NT
// threads (E <= INLINE_E <= NT; a wave per token reads its logits from
// global memory); workgroup (0,0,0) also publishes them for the later
// kernels.  Results land in the LDS arrays of `R`.  With T = 1
// there is no grouping: slot j of the token is a group of its own.
struct alignas(16) InlineRoute {
	float w[INLINE_T * MAX_K];
	int32_t idx[INLINE_T * MAX_K];
	alignas(16) int32_t cnt[INLINE_E];
	int32_t cur[INLINE_E];
	int32_t offsets[INLINE_E + 1], active[INLINE_E + 1];
	int32_t pairs[INLINE_T * MAX_K];
	int wsum[16];
	uint64_t etab[32];
};

template <int NT> __device__ __forceinline__ void inline_route(const ExactArgs &a, InlineRoute &R)
{
	const int tid = threadIdx.x;
	const int T = a.T, E = a.E, k = a.k;
	if (tid < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		R.etab[tid] = tab[tid];
	}
	__syncthreads();
	for (int t = tid >> 6; t < T; t += NT / 64)
		topk_softmax_wave<INLINE_E / 64>(a.logits + (size_t)t * E, E, k, R.etab, R.idx + t * k, R.w + t * k,
						 a.routing, a.pbias);
	__syncthreads();
	if (a.single) {
		// one token: slot j is its own group (expert idx[j], pair j); the
		// later kernels of this mode read only the selection
		if (tid < k)
			R.pairs[tid] = tid;
		if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && tid < k) {
			a.topk_idx[tid] = R.idx[tid];
			a.topk_w[tid] = R.w[tid];
		}
		__syncthreads();
		return;
	}
	// every workgroup groups on its own and must reach the same expert order:
	// ascending expert index (the count order breaks ties by LDS atomics)
	group_pairs<NT>(R.idx, T * k, E, R.cnt, R.cur, R.wsum, R.offsets, R.pairs, R.active);
	if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) {
		for (int i = tid; i < T * k; i += NT) {
			a.topk_idx[i] = R.idx[i];
			a.topk_w[i] = R.w[i];
			a.pairs[i] = R.pairs[i];
		}
		for (int i = tid; i <= E; i += NT) {
			a.offsets[i] = R.offsets[i];
			a.active[i] = R.active[i];
		}
	}
}

// ------------------------------------------------------------ gate / up
// blockIdx = (64-row panel, active-expert slot, matrix).  FUSED: one
// workgroup per (panel, slot) runs both matrices (wave w: gate and up
// column w, w + 8, ..) and applies TIE's table SwiGLU
// (swiglu_activation_f32_f32_avx2) to the row sums, writing h; otherwise
// blockIdx.z selects the matrix and the row sums are written.
template <int TYPE, bool FUSED, int PM>
__global__ __launch_bounds__(GU_THREADS) GU_OCC void exact_gu_kernel(ExactArgs a)
{
	// fused: as many waves as the launch chose; split: GU_WAVES
	const int NW = FUSED ? __builtin_amdgcn_readfirstlane(blockDim.x >> 6) : GU_WAVES;
	using Block = typename BlockOf<TYPE>::type;
	extern __shared__ float part[]; // [mats][nb][pg_cap][64]
	const int32_t *offsets = a.offsets, *pairs = a.pairs, *active = a.active;
	const int32_t *sel_idx = nullptr;
	if constexpr (!FUSED) {
		// the fused kernel never routes inline: no LDS reserved for it
		__shared__ InlineRoute R;
		if (a.inline_route) {
			inline_route<GU_THREADS>(a, R);
			offsets = R.offsets;
			pairs = R.pairs;
			active = R.active;
			sel_idx = R.idx;
		}
	}
	auto single_expert = [&](const ExactArgs &, const int32_t *, int j) { return j < a.k ? sel_idx[j] : -1; };
	const int slot = blockIdx.y;
	int e, p0, p1;
	if (!FUSED && a.single) {
		// one token: the slot's selected expert, the slot's own pair
		e = __builtin_amdgcn_readfirstlane(single_expert(a, pairs, slot));
		if (e < 0)
			return;
		p0 = slot;
		p1 = slot + 1;
	} else {
		if (slot >= active[a.E])
			return;
		e = active[slot];
		p0 = offsets[e];
		p1 = offsets[e + 1];
	}
	const int rt = blockIdx.x;
	const int lane = threadIdx.x & 63;
	const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int nb = a.in / QK;
	const int nmat = FUSED ? 2 : 1;
	const int m0 = FUSED ? 0 : (int)blockIdx.z;
	const size_t pb = panel_bytes(TYPE);
	const int pg_cap = a.pg_cap;
	const int k = a.k, in = a.in;
	const float *x = a.x;

	for (int g0 = p0; g0 < p1; g0 += pg_cap) {
		const int np = min(pg_cap, p1 - g0);
		const int32_t *gp = pairs + g0;
		const int ntask = nmat * nb;
		auto panel_of = [&](int t) {
			const int mi = t / nb, b = t - mi * nb;
			return a.w[m0 + mi] + (size_t)e * a.expert_bytes[m0 + mi] + ((size_t)rt * nb + b) * pb;
		};
		for (int t = w; t < ntask; t += NW) {
			const int b = t % nb;
			Block blk;
			load_block(panel_of(t), lane, blk);
			auto xrow_b = [&](int q) {
				const int pair = __builtin_amdgcn_readfirstlane(gp[q]);
				return (cfloat *)(x + (size_t)(pair / k) * in + QK * b);
			};
			block_all_pairs<PM, Block, cfloat>(blk, np, xrow_b, part + (size_t)t * pg_cap * 64, lane);
		}
		__syncthreads();
		// serial sums over super-blocks (math_avx2.c:762-766)
		for (int i = threadIdx.x; i < np * 64; i += 64 * NW) {
			const int q = i >> 6, r = i & 63;
			const size_t o = (size_t)gp[q] * a.rows + rt * PANEL_ROWS + r;
			float s0 = 0.0f;
			for (int b = 0; b < nb; b++)
				s0 = s0 + part[((size_t)b * pg_cap + q) * 64 + r];
			if (FUSED) {
				float s1 = 0.0f;
				for (int b = 0; b < nb; b++)
					s1 = s1 + part[((size_t)(nb + b) * pg_cap + q) * 64 + r];
				a.hbuf[o] = tie_swiglu(s0, s1, a.silu);
			} else {
				a.sums[m0][o] = s0;
			}
		}
		__syncthreads();
	}
}

// BF16 gate/up: mat_vec_row_f32_bf16_f32_avx2 + dot_product_f32_bf16_avx2
// (math_avx2.c:148-158, 188-226): 8 lane accumulators over the whole row,
// then hsum8.  Thread h of a row owns lanes 4h..4h+3.
constexpr int BF_THREADS = 128;
__global__ __launch_bounds__(BF_THREADS) void exact_gu_bf16_kernel(ExactArgs a)
{
	__shared__ InlineRoute R;
	const int32_t *offsets = a.offsets, *pairs = a.pairs, *active = a.active;
	if (a.inline_route) {
		inline_route<BF_THREADS>(a, R);
		offsets = R.offsets;
		pairs = R.pairs;
		active = R.active;
	}
	const int slot = blockIdx.y;
	if (slot >= active[a.E])
		return;
	const int m = blockIdx.z;
	const int e = active[slot];
	const int p0 = offsets[e], p1 = offsets[e + 1];
	const int r = threadIdx.x >> 1, h = threadIdx.x & 1;
	const int row = blockIdx.x * PANEL_ROWS + r;
	const uint16_t *wr = reinterpret_cast<const uint16_t *>(a.w[m] + (size_t)e * a.expert_bytes[m]) +
			     (size_t)row * a.in;
	for (int p = p0; p < p1; p++) {
		const int pair = pairs[p];
		const float *xin = a.x + (size_t)(pair / a.k) * a.in;
		float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
		for (int i = 0; i < a.in; i += 8) {
			const uint2 wv = *reinterpret_cast<const uint2 *>(wr + i + 4 * h);
			const float4 xv = *reinterpret_cast<const float4 *>(xin + i + 4 * h);
			acc[0] = __builtin_fmaf(xv.x, bf16_bits_to_float(wv.x & 0xffffu), acc[0]);
			acc[1] = __builtin_fmaf(xv.y, bf16_bits_to_float(wv.x >> 16), acc[1]);
			acc[2] = __builtin_fmaf(xv.z, bf16_bits_to_float(wv.y & 0xffffu), acc[2]);
			acc[3] = __builtin_fmaf(xv.w, bf16_bits_to_float(wv.y >> 16), acc[3]);
		}
		// s_m = v[m] + v[m+4] (m = 0..3 on h = 0), then (s0+s1)+(s2+s3)
		float o[4];
#pragma unroll
		for (int i = 0; i < 4; i++)
			o[i] = __shfl_xor(acc[i], 1);
		const float s0 = acc[0] + o[0], s1 = acc[1] + o[1], s2 = acc[2] + o[2], s3 = acc[3] + o[3];
		if (h == 0)
			a.sums[m][(size_t)pair * a.rows + row] = (s0 + s1) + (s2 + s3);
	}
}

// ------------------------------------------------------------ down
// h = silu_tab(gate) * up for the np pairs of a group, into LDS [np][F]
__device__ __forceinline__ void stage_h(const ExactArgs &a, const int32_t *gp, int np, float *hs)
{
	const int F = a.in;
	for (int i = threadIdx.x; i < np * F; i += blockDim.x) {
		const int q = i / F, f = i - q * F;
		const size_t o = (size_t)gp[q] * F + f;
		hs[i] = tie_swiglu(a.sums[0][o], a.sums[1][o], a.silu);
	}
}

// blockIdx = (64-row panel of d, active-expert slot); blockDim = 64 * nb
// up to nb = 6, else 64 * min(ceil(nb / 2), 8) (waves stride the blocks).  HG: h comes from hbuf (written by the fused gate/up kernel)
// through scalar loads; otherwise the prologue forms h from the gate and up
// row sums in LDS.  Dynamic LDS: [h [pg_cap][F] |] part [nb][pg_cap][64].
template <int TYPE, bool HG, int PM>
__global__ __launch_bounds__(512) EXACT_OCC void exact_down_kernel(ExactArgs a)
{
	using Block = typename BlockOf<TYPE>::type;
	extern __shared__ float lds[];
	const int slot = blockIdx.y;
	int e, p0, p1;
	const int32_t *pairs = a.pairs;
	if (a.single) {
		// one token: the slot's selected expert and its own pair
		e = slot < a.k ? a.topk_idx[slot] : -1;
		if (e < 0)
			return;
		p0 = slot;
		p1 = slot + 1;
		pairs = nullptr;
	} else {
		if (slot >= a.active[a.E])
			return;
		e = a.active[slot];
		p0 = a.offsets[e];
		p1 = a.offsets[e + 1];
	}
	const int rt = blockIdx.x;
	const int lane = threadIdx.x & 63;
	const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int nw = blockDim.x >> 6;
	const int F = a.in, nb = F / QK;
	const size_t pb = panel_bytes(TYPE);
	const uint8_t *panels = a.w[0] + (size_t)e * a.expert_bytes[0] + (size_t)rt * nb * pb;
	const int pg_cap = a.pg_cap;
	float *hs = lds;
	float *part = HG ? lds : lds + (size_t)pg_cap * F;

	// single mode: the group is the slot's own pair, listed in LDS
	__shared__ int32_t own_pair[1];
	if (!pairs) {
		own_pair[0] = p0;
		__syncthreads();
	}
	for (int g0 = p0; g0 < p1; g0 += pg_cap) {
		const int np = min(pg_cap, p1 - g0);
		const int32_t *gp = pairs ? pairs + g0 : own_pair;
		if (!HG) {
			stage_h(a, gp, np, hs);
			__syncthreads();
		}
		for (int b = w; b < nb; b += nw) {
			Block blk;
			load_block(panels + (size_t)b * pb, lane, blk);
			if (HG) {
				auto xrow_b = [&](int q) {
					const int pair = __builtin_amdgcn_readfirstlane(gp[q]);
					return (cfloat *)(a.hbuf + (size_t)pair * F + QK * b);
				};
				block_all_pairs<PM, Block, cfloat>(blk, np, xrow_b, part + (size_t)b * pg_cap * 64, lane);
			} else {
				auto xrow_b = [&](int q) { return (lfloat *)(hs + (size_t)q * F + QK * b); };
				block_all_pairs<PM, Block, lfloat>(blk, np, xrow_b, part + (size_t)b * pg_cap * 64, lane);
			}
		}
		__syncthreads();
		for (int i = threadIdx.x; i < np * 64; i += blockDim.x) {
			const int q = i >> 6, r = i & 63;
			float s = 0.0f;
			for (int b = 0; b < nb; b++)
				s = s + part[((size_t)b * pg_cap + q) * 64 + r];
			a.y[(size_t)gp[q] * a.rows + rt * PANEL_ROWS + r] = s;
		}
		__syncthreads();
	}
}

// BF16 down: blockIdx = (64-row panel of d, slot), 128 threads.  Dynamic
// LDS: h [pg_cap][F].
__global__ __launch_bounds__(BF_THREADS) void exact_down_bf16_kernel(ExactArgs a)
{
	extern __shared__ float hs[];
	const int slot = blockIdx.y;
	if (slot >= a.active[a.E])
		return;
	const int e = a.active[slot];
	const int p0 = a.offsets[e], p1 = a.offsets[e + 1];
	const int r = threadIdx.x >> 1, h = threadIdx.x & 1;
	const int row = blockIdx.x * PANEL_ROWS + r;
	const int F = a.in;
	const uint16_t *wr = reinterpret_cast<const uint16_t *>(a.w[0] + (size_t)e * a.expert_bytes[0]) +
			     (size_t)row * F;
	const int pg_cap = a.pg_cap;
	for (int g0 = p0; g0 < p1; g0 += pg_cap) {
		const int np = min(pg_cap, p1 - g0);
		const int32_t *gp = a.pairs + g0;
		stage_h(a, gp, np, hs);
		__syncthreads();
		for (int q = 0; q < np; q++) {
			const float *xin = hs + (size_t)q * F;
			float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
			for (int i = 0; i < F; i += 8) {
				const uint2 wv = *reinterpret_cast<const uint2 *>(wr + i + 4 * h);
				const float4 xv = *reinterpret_cast<const float4 *>(xin + i + 4 * h);
				acc[0] = __builtin_fmaf(xv.x, bf16_bits_to_float(wv.x & 0xffffu), acc[0]);
				acc[1] = __builtin_fmaf(xv.y, bf16_bits_to_float(wv.x >> 16), acc[1]);
				acc[2] = __builtin_fmaf(xv.z, bf16_bits_to_float(wv.y & 0xffffu), acc[2]);
				acc[3] = __builtin_fmaf(xv.w, bf16_bits_to_float(wv.y >> 16), acc[3]);
			}
			float o[4];
#pragma unroll
			for (int i = 0; i < 4; i++)
				o[i] = __shfl_xor(acc[i], 1);
			const float s0 = acc[0] + o[0], s1 = acc[1] + o[1], s2 = acc[2] + o[2], s3 = acc[3] + o[3];
			if (h == 0)
				a.y[(size_t)gp[q] * a.rows + row] = (s0 + s1) + (s2 + s3);
		}
		__syncthreads();
	}
}

// ---------------------------------------------------------------- launcher
// Raise a kernel's dynamic-LDS limit to at least `bytes`.  The limit is
// remembered per kernel, so the attribute call (host work on every launch
// otherwise) happens only when a launch needs more than before.
hipError_t ensure_lds_limit(const void *fn, size_t bytes)
{
	static std::unordered_map<const void *, size_t> limit;
	auto it = limit.find(fn);
	if (it != limit.end() && it->second >= bytes)
		return hipSuccess;
	const hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
	if (err == hipSuccess)
		limit[fn] = bytes;
	return err;
}

static hipError_t set_lds_limit(const void *fn, size_t bytes)
{
	return ensure_lds_limit(fn, bytes);
}

static int clamp_pg(int v)
{
	return v > PG_MAX ? PG_MAX : v < 1 ? 1 : v;
}

// Launch a quantised kernel template instance with `lds` bytes of dynamic
// LDS (raising the function's limit first).
template <typename K>
static hipError_t launch_q(K kernel, dim3 grid, dim3 block, size_t lds, size_t static_lds, hipStream_t s,
			   const ExactArgs &a)
{
	hipError_t err = set_lds_limit((const void *)kernel, lds + static_lds);
	if (err != hipSuccess)
		return err;
	tie_launch(kernel, grid, block, lds, s, a);
	return hipGetLastError();
}

// Waves per workgroup for a launch of n_wg workgroups that each run `tasks`
// super-block columns, wave w taking columns w, w + nw, ..: the count in
// [1, 8] that minimises rounds * ceil(tasks / nw), where a round is one
// workgroup on every resident slot of the chip (the occupancy API's
// workgroups per CU, which counts registers and LDS, times the CUs).  The
// grids here are often only slightly larger than one round, so a wave count
// that packs more workgroups per CU, or gives each fewer columns, shortens
// the last, partly filled round.  Ties go to more waves (at most `tasks`).
static int pick_waves_uncached(const void *fn, size_t lds, int n_wg, int tasks)
{
	static int ncu = 0;
	if (!ncu) {
		int dev = 0;
		if (hipGetDevice(&dev) != hipSuccess ||
		    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
			ncu = 256;
	}
	const int wmax = tasks < 8 ? tasks : 8;
	int best = wmax;
	long best_cost = -1;
	for (int w = wmax; w >= 1; w--) {
		int occ = 0;
		if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, 64 * w, lds) != hipSuccess || occ <= 0)
			continue;
		const long slots = (long)ncu * occ;
		const long cost = (long)((n_wg + slots - 1) / slots) * ((tasks + w - 1) / w);
		if (best_cost < 0 || cost < best_cost) {
			best_cost = cost;
			best = w;
		}
	}
	return best;
}

// pick_waves, memoised (the occupancy queries are host work)
static int pick_waves(const void *fn, size_t lds, int n_wg, int tasks)
{
	static std::map<std::tuple<const void *, size_t, int, int>, int> memo;
	const auto key = std::make_tuple(fn, lds, n_wg, tasks);
	auto it = memo.find(key);
	if (it != memo.end())
		return it->second;
	const int w = pick_waves_uncached(fn, lds, n_wg, tasks);
	memo[key] = w;
	return w;
}

// Expected number of experts with at least one pair: E (1 - (1 - k/E)^T)
// for independent uniform selections, at most max_active.
static int expected_active(int E, int k, int T, int max_active)
{
	const double a = E * (1.0 - std::pow(1.0 - (double)k / E, (double)T));
	const int n = (int)std::ceil(a);
	return n < 1 ? 1 : n > max_active ? max_active : n;
}

// gate/up of one quantised type; fused (both matrices, h out) or one
// matrix per blockIdx.z (row sums out)
static hipError_t launch_gu_q(int type, bool fused, int nmat, int rows, int in, int max_active, ExactArgs g,
			      hipStream_t s)
{
	const int nb = in / QK;
	const int mats = fused ? 2 : 1;
	// small pair groups: the LDS of a workgroup stays small enough for
	// several workgroups per CU (experts with more pairs run more groups)
	g.pg_cap = clamp_pg(PART_FLOATS / (mats * nb * 64));
	if (g.pg_cap > TIE_GU_PG)
		g.pg_cap = TIE_GU_PG;
	g.rows = rows;
	g.in = in;
	const size_t lds = sizeof(float) * (size_t)mats * nb * g.pg_cap * 64;
	const dim3 grid(rows / PANEL_ROWS, max_active, fused ? 1 : nmat);
	dim3 block(64 * GU_WAVES);
	const size_t st = fused ? 0 : sizeof(InlineRoute);
	constexpr int PM = TIE_EXACT_PCMAX;
	// one token (one pair per group): a one-pair instance, whose register
	// budget, and so occupancy, is not set by the multi-pair dot products
	if (g.single)
		return type == TIE_GGML_Q4_K ? launch_q(exact_gu_kernel<TIE_GGML_Q4_K, false, 1>, grid, block, lds, st, s, g)
					     : launch_q(exact_gu_kernel<TIE_GGML_Q6_K, false, 1>, grid, block, lds, st, s, g);
	if (fused) {
		const void *fn = type == TIE_GGML_Q4_K ? (const void *)exact_gu_kernel<TIE_GGML_Q4_K, true, PM>
						      : (const void *)exact_gu_kernel<TIE_GGML_Q6_K, true, PM>;
		hipError_t err = set_lds_limit(fn, lds);
		if (err != hipSuccess)
			return err;
		block.x = 64 * pick_waves(fn, lds, (rows / PANEL_ROWS) * expected_active(g.E, g.k, g.T, max_active),
					  2 * nb);
	}
	if (type == TIE_GGML_Q4_K)
		return fused ? launch_q(exact_gu_kernel<TIE_GGML_Q4_K, true, PM>, grid, block, lds, st, s, g)
			     : launch_q(exact_gu_kernel<TIE_GGML_Q4_K, false, PM>, grid, block, lds, st, s, g);
	return fused ? launch_q(exact_gu_kernel<TIE_GGML_Q6_K, true, PM>, grid, block, lds, st, s, g)
		     : launch_q(exact_gu_kernel<TIE_GGML_Q6_K, false, PM>, grid, block, lds, st, s, g);
}

// Routing (logits, selection, grouping) and the expert GEMVs of the exact
// path.  ws.h holds two [pairs][F] planes: the gate and the up row sums, or
// (fused gate/up) h in the first.
hipError_t launch_exact_block(const Layer &L, const float *x, int T, int k, const float *silu, Workspace &ws,
			      float *out, hipStream_t s, const float *res)
{
	const int npairs = T * k;
	if (npairs == 0)
		return hipSuccess;
	const int max_active = npairs < L.E ? npairs : L.E;
	hipError_t err;
	prof_begin("router", s);
	err = launch_router_logits(L, x, T, ws.logits, s);
	prof_end(s);
	if (err != hipSuccess)
		return err;
	const bool same = L.gate.type == L.up.type;
	const bool quant = L.gate.type != TIE_GGML_BF16 && L.up.type != TIE_GGML_BF16;
	const bool inl = T <= INLINE_T && L.E <= INLINE_E && same;
	// Small T: gate and up in separate workgroups (twice the parallelism),
	// h formed in the down prologue.  Otherwise one workgroup per panel runs
	// both and writes h, which the down kernel reads through scalar loads.
	const bool fused = !inl && same && quant && L.down.type != TIE_GGML_BF16;
	// one token: slot j is pair j of expert topk_idx[j]; no grouping
	const bool single = T == 1 && inl && quant && L.down.type != TIE_GGML_BF16;
	if (!inl) {
		prof_begin("route_group", s);
		if (npairs <= 4096)
			err = launch_route_group(L, T, k, ws.logits, ws, s);
		else {
			err = launch_router_select(L, T, k, ws.logits, ws.topk_idx, ws.topk_w, s);
			if (err == hipSuccess)
				err = launch_dispatch(L, T, k, ws.topk_idx, ws, s);
		}
		prof_end(s);
		if (err != hipSuccess)
			return err;
	}
	ExactArgs a;
	memset(&a, 0, sizeof a);
	a.k = k;
	a.E = L.E;
	a.T = T;
	a.x = x;
	a.sums[0] = ws.h;
	a.sums[1] = ws.h + (size_t)npairs * L.F;
	a.hbuf = ws.h;
	a.y = ws.y;
	a.silu = silu;
	a.logits = ws.logits;
	a.topk_idx = ws.topk_idx;
	a.topk_w = ws.topk_w;
	a.offsets = ws.offsets;
	a.pairs = ws.pairs;
	a.active = ws.active;
	a.inline_route = inl ? 1 : 0;
	a.routing = L.routing;
	a.pbias = L.pbias;
	a.single = single ? 1 : 0;

	prof_begin("exact_gate_up", s);
	{
		ExactArgs g = a;
		g.w[0] = L.gate.data;
		g.w[1] = L.up.data;
		g.expert_bytes[0] = L.gate.expert_bytes;
		g.expert_bytes[1] = L.up.expert_bytes;
		if (same && L.gate.type == TIE_GGML_BF16) {
			g.rows = L.F;
			g.in = L.d;
			tie_launch(exact_gu_bf16_kernel, dim3(L.F / PANEL_ROWS, max_active, 2), dim3(BF_THREADS), 0,
					   s, g);
			err = hipGetLastError();
		} else if (same) {
			err = launch_gu_q(L.gate.type, fused, 2, L.F, L.d, max_active, g, s);
		} else {
			// gate and up of different types: one launch per matrix, each
			// with its matrix in slot 0 of the arguments
			for (int mat = 0; mat < 2 && err == hipSuccess; mat++) {
				const ExpertTensor &t = mat == 0 ? L.gate : L.up;
				ExactArgs h = g;
				h.w[0] = t.data;
				h.expert_bytes[0] = t.expert_bytes;
				h.sums[0] = a.sums[mat];
				if (t.type == TIE_GGML_BF16) {
					h.rows = t.rows;
					h.in = t.in;
					tie_launch(exact_gu_bf16_kernel, dim3(t.rows / PANEL_ROWS, max_active, 1),
							   dim3(BF_THREADS), 0, s, h);
					err = hipGetLastError();
				} else {
					err = launch_gu_q(t.type, false, 1, t.rows, t.in, max_active, h, s);
				}
			}
		}
	}
	prof_end(s);
	if (err != hipSuccess)
		return err;

	prof_begin("exact_down", s);
	{
		constexpr int PM = TIE_EXACT_PCMAX;
		ExactArgs g = a;
		g.w[0] = L.down.data;
		g.expert_bytes[0] = L.down.expert_bytes;
		g.rows = L.d;
		g.in = L.F;
		const dim3 grid(L.d / PANEL_ROWS, max_active);
		const int F = L.F, nb = F / QK;
		if (L.down.type == TIE_GGML_BF16) {
			g.pg_cap = clamp_pg(PART_FLOATS / F);
			const size_t lds = sizeof(float) * (size_t)g.pg_cap * F;
			err = launch_q(exact_down_bf16_kernel, grid, dim3(BF_THREADS), lds, 0, s, g);
		} else {
			dim3 block(64);
			const int n_wg = (L.d / PANEL_ROWS) * expected_active(L.E, k, T, max_active);
			if (fused) {
				g.pg_cap = clamp_pg(PART_FLOATS / (nb * 64));
				const size_t lds = sizeof(float) * (size_t)g.pg_cap * nb * 64;
				// pairs dequantised together: 2 where experts average at
				// most 4 pairs (92 instead of 125 registers: 5 waves per
				// SIMD instead of 4), else PM
				auto run = [&](auto pmc) -> hipError_t {
					constexpr int P = decltype(pmc)::value;
					const void *fn = L.down.type == TIE_GGML_Q4_K ? (const void *)exact_down_kernel<TIE_GGML_Q4_K, true, P>
										       : (const void *)exact_down_kernel<TIE_GGML_Q6_K, true, P>;
					hipError_t e2 = set_lds_limit(fn, lds);
					if (e2 != hipSuccess)
						return e2;
					block.x = 64 * pick_waves(fn, lds, n_wg, nb);
					return L.down.type == TIE_GGML_Q4_K
						       ? launch_q(exact_down_kernel<TIE_GGML_Q4_K, true, P>, grid, block, lds, 0, s, g)
						       : launch_q(exact_down_kernel<TIE_GGML_Q6_K, true, P>, grid, block, lds, 0, s, g);
				};
				if (TIE_DOWN_PM2 && (long)T * k <= 4L * L.E)
					err = run(std::integral_constant<int, 2>{});
				else
					err = run(std::integral_constant<int, PM>{});
			} else {
				g.pg_cap = clamp_pg(PART_FLOATS / (F + nb * 64));
				const size_t lds = sizeof(float) * (size_t)g.pg_cap * (F + nb * 64);
				const void *fn = single ? (L.down.type == TIE_GGML_Q4_K
								   ? (const void *)exact_down_kernel<TIE_GGML_Q4_K, false, 1>
								   : (const void *)exact_down_kernel<TIE_GGML_Q6_K, false, 1>)
							: (L.down.type == TIE_GGML_Q4_K
								   ? (const void *)exact_down_kernel<TIE_GGML_Q4_K, false, PM>
								   : (const void *)exact_down_kernel<TIE_GGML_Q6_K, false, PM>);
				err = set_lds_limit(fn, lds);
				if (err != hipSuccess)
					return err;
				block.x = 64 * pick_waves(fn, lds, single ? (L.d / PANEL_ROWS) * k : n_wg, nb);
				if (single)
					err = L.down.type == TIE_GGML_Q4_K
						      ? launch_q(exact_down_kernel<TIE_GGML_Q4_K, false, 1>, grid, block, lds, 0, s, g)
						      : launch_q(exact_down_kernel<TIE_GGML_Q6_K, false, 1>, grid, block, lds, 0, s, g);
				else
					err = L.down.type == TIE_GGML_Q4_K
						      ? launch_q(exact_down_kernel<TIE_GGML_Q4_K, false, PM>, grid, block, lds, 0, s, g)
						      : launch_q(exact_down_kernel<TIE_GGML_Q6_K, false, PM>, grid, block, lds, 0, s, g);
			}
		}
	}
	prof_end(s);
	if (err != hipSuccess)
		return err;
	prof_begin("combine", s);
	err = launch_combine(T, L.d, k, ws.topk_w, ws.topk_idx, ws.y, out, s, res);
	prof_end(s);
	return err;
}

// ------------------------------------------------------------ dense
// dispatch_mat_mat (math_dispatch.c:304-359) with F32 input: every token row
// through the same row kernel as the experts (mat_vec_row_f32_{q4k,q6k,
// bf16}_f32_avx2), so the expert GEMV kernels run it unchanged: the tokens
// are split into groups of DENSE_GROUP, and each group is an "expert" of
// stride 0 (every group reads the one matrix), so groups spread over the
// grid's y dimension and each workgroup computes one 64-row panel for one
// group.  out[t][r], [T][rows].
constexpr int DENSE_GROUP = 8;

__global__ void dense_groups_kernel(int T, int G, int32_t *offsets, int32_t *pairs, int32_t *active)
{
	const int i = blockIdx.x * blockDim.x + threadIdx.x;
	if (i < T)
		pairs[i] = i;
	if (i <= G) {
		offsets[i] = i * DENSE_GROUP < T ? i * DENSE_GROUP : T;
		active[i] = i < G ? i : G;
	}
}

int dense_groups(int T)
{
	return (T + DENSE_GROUP - 1) / DENSE_GROUP;
}

hipError_t launch_dense(const ExpertTensor &W, const float *x, int T, float *out, Workspace &ws, hipStream_t s)
{
	if (T == 0)
		return hipSuccess;
	const int G = dense_groups(T);
	tie_launch(dense_groups_kernel, dim3((T + 1 + 255) / 256 > (G + 1 + 255) / 256 ? (T + 1 + 255) / 256
											  : (G + 1 + 255) / 256),
			   dim3(256), 0, s, T, G, ws.offsets, ws.pairs, ws.active);
	hipError_t err = hipGetLastError();
	if (err != hipSuccess)
		return err;
	ExactArgs a;
	memset(&a, 0, sizeof a);
	a.w[0] = W.data;
	a.expert_bytes[0] = 0;
	a.k = 1;
	a.E = G;
	a.T = T;
	a.x = x;
	a.sums[0] = out;
	a.offsets = ws.offsets;
	a.pairs = ws.pairs;
	a.active = ws.active;
	a.rows = W.rows;
	a.in = W.in;
	if (W.type == TIE_GGML_BF16) {
		tie_launch(exact_gu_bf16_kernel, dim3(W.rows / PANEL_ROWS, G, 1), dim3(BF_THREADS), 0, s, a);
		return hipGetLastError();
	}
	return launch_gu_q(W.type, false, 1, W.rows, W.in, G, a, s);
}

} // namespace tie
