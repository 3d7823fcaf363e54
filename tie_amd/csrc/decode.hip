// decode.hip -- the block for one token at a time, in TIE's exact fp32
// arithmetic: decode (T = 1), and the exact recomputation of listed tokens
// of a large-T forward (tokens whose activations left the f16 range of the
// matrix-core path).
//
// Reference: per token, TIE runs k process_expert_task jobs
// (engine.c:916-964): gate and up GEMVs (mat_vec_row_f32_{q4k,q6k}_f32_avx2,
// math_avx2.c:753-787, a serial fp32 sum over the row's super-block dots
// dot_product_f32_{q4k,q6k}_avx2, :535-604 / :411-495), the table SwiGLU
// (swiglu_activation_f32_f32_avx2, :908-950) and the down GEMV, then the
// combine out = sum_j g_j y_j in slot order (model_qwen3.c:459-467).
//
// At one token nothing is shared between the k experts, so the work is a
// set of independent (row, super-block) dot products.  Each lane owns one:
// it issues the loads of its whole block (Q4_K 9, Q6_K 13 chunks of 16
// bytes, all in flight at once) and runs TIE's dot with the input vector
// read from LDS.  A workgroup holds every block of R rows, so the serial
// per-row sums over the blocks, the SwiGLU (gate/up) and the combine over
// the k experts (down) happen in its epilogue without another launch:
//
//   decode_gu_kernel    blockIdx = (R rows of F, slot j, list entry);
//                       lane = (row, matrix, block): 2 nb R dots.  Writes
//                       h = silu_tab(gate) * up of the slot's expert.
//   decode_down_kernel  blockIdx = (R rows of d, -, list entry);
//                       lane = (row, slot, block): k nb R dots.  Writes
//                       out = [res +] sum_j g_j y_j, i.e. the combine.
//
// Rows are read from the panel layout (common.h): rows r0..r0+R-1 of a
// panel are R consecutive 16-byte slots of every 1 KiB chunk.  The input
// vector (x, or the k h vectors) sits in LDS as 256-float segments, each
// padded by XPAD floats so that the segments a wave reads at once start in
// different banks.
#include "common.h"
#include "route.h"

#include <algorithm>

namespace tie {

constexpr int XPAD = 4;
constexpr int INLINE_E = 128; // inline routing: experts held by one wave (two per lane)

// LDS scratch of topk_softmax_block for E <= INLINE_E
struct TopkScratch {
	alignas(16) uint32_t key[INLINE_E];
	float prob[INLINE_E];
	int rank[INLINE_E];
	float sv[MAX_K];
	int si[MAX_K];
}; // gate/up workgroups of the one-launch decode at most (done words)
constexpr int XSEG = QK + XPAD;
constexpr int DEC_MAX_THREADS = 512;
// waves per SIMD the registers of the one-launch decode's two-lane form
// leave room for (its workgroups must all be resident at once)
constexpr int ONE_PAIR_WAVES = 6;
constexpr size_t DEC_MAX_LDS = 150 * 1024; // dynamic LDS per workgroup at most (160 KiB per CU)

typedef const float __attribute__((address_space(3))) dfloat; // LDS input rows
typedef float vf4 __attribute__((ext_vector_type(4)));
typedef const vf4 __attribute__((address_space(3))) dfloat4;

__device__ __forceinline__ uint32_t dword_of(const uint4 &v, int i)
{
	return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Make v opaque at this point of the instruction stream: the work that
// depends on it cannot be hoisted above (the block's chunks are all loaded
// up front, so without these the scheduler would dequantise the whole block
// at once and run out of registers).
__device__ __forceinline__ void pin(uint4 &v)
{
	asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// Accumulator fence: an empty statement that reads and writes all 16
// accumulators, so it cannot run before the FMAs issued ahead of it.  The
// pins that follow it (volatile statements keep their order) therefore
// hold the next group's work behind the previous group's FMAs.
__device__ __forceinline__ void acc_fence(float (&a0)[8], float (&a1)[8])
{
	asm volatile("" : "+v"(a0[0]), "+v"(a0[1]), "+v"(a0[2]), "+v"(a0[3]), "+v"(a0[4]), "+v"(a0[5]), "+v"(a0[6]),
			  "+v"(a0[7]));
	asm volatile("" : "+v"(a1[0]), "+v"(a1[1]), "+v"(a1[2]), "+v"(a1[3]), "+v"(a1[4]), "+v"(a1[5]), "+v"(a1[6]),
			  "+v"(a1[7]));
}

__device__ __forceinline__ float byte_f(uint32_t w, int i)
{
	return (float)((w >> (8 * i)) & 0xffu);
}

// get_scale_min_k4 (math_scalar.c:91-100) of sub-block j: D = d * sc,
// nM = -(dmin * m)
__device__ __forceinline__ void q4k_scale(const uint4 &c0, int j, float d, float dmin, float &D, float &nM)
{
	const uint32_t s[3] = {c0.y, c0.z, c0.w};
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

// dot_product_f32_q4k_avx2 (math_avx2.c:535-604) of one block (chunks c[0..8]
// of the panel layout: c[0] = d, dmin, scales; c[1 + 2g + o] = code bytes
// 64g + 16o .. +15) with 256 inputs x.  16 accumulators (two 8-lane AVX2
// registers): weight w = fma(q, d*sc, -(dmin*m)); step (g, o, h) covers
// codes 64g + 16o + 4h + i (low nibbles: x[64g + 16o + 4h + i], high: +32),
// accumulator 4h + i; then lo + hi and hsum_f32_avx2.
__device__ __forceinline__ float q4k_dot(uint4 (&c)[9], dfloat *x)
{
	const float d = half_bits_to_float(c[0].x & 0xffffu);
	const float dmin = half_bits_to_float(c[0].x >> 16);
	float a0[8], a1[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		a0[l] = a1[l] = 0.0f;
#pragma unroll
	for (int g = 0; g < 4; g++) {
		// one 64-weight group at a time
		acc_fence(a0, a1);
		asm volatile("" : "+v"(x));
		pin(c[1 + 2 * g]);
		pin(c[2 + 2 * g]);
		float D1, M1, D2, M2;
		q4k_scale(c[0], 2 * g, d, dmin, D1, M1);
		q4k_scale(c[0], 2 * g + 1, d, dmin, D2, M2);
#pragma unroll
		for (int ss = 0; ss < 8; ss++) {
			const int o = ss >> 2, h = ss & 3;
			const uint32_t w = dword_of(c[1 + 2 * g + o], h);
			uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
			// byte-parallel words: each code is then one v_cvt_f32_ubyteN
			asm volatile("" : "+v"(lo), "+v"(hi));
			dfloat *xb = x + 64 * g + 16 * o + 4 * h;
			const vf4 xl = *(dfloat4 *)xb, xh = *(dfloat4 *)(xb + 32);
			const float xlv[4] = {xl.x, xl.y, xl.z, xl.w}, xhv[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
			for (int i = 0; i < 4; i++) {
				const float wl = __builtin_fmaf(byte_f(lo, i), D1, M1);
				const float wh = __builtin_fmaf(byte_f(hi, i), D2, M2);
				const int m = 4 * h + i;
				float &A = (m < 8) ? a0[m & 7] : a1[m & 7];
				A = __builtin_fmaf(xlv[i], wl, A);
				A = __builtin_fmaf(xhv[i], wh, A);
			}
		}
	}
	float v[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		v[l] = a0[l] + a1[l];
	return hsum8(v);
}

// dot_product_f32_q6k_avx2 (math_avx2.c:411-495) of one block (chunks
// c[0..12] of the panel layout: 0-7 ql, 8-11 qh, 12 the int8 scales; d
// the fp16 scale) with 256 inputs x.  Step (n, l, hw) forms the codes
// q = ql nibble | qh bits << 4 of weights 128n + l + 4hw + i + 32r (r =
// 0..3) and accumulates fma(d*sc, (q - 32) * x, acc) into accumulators
// 4hw + i of a0 (r = 0, 2) and a1 (r = 1, 3), the product rounded on its
// own.  PX: the input pairs of each half step are read from LDS one half
// step ahead (streamed kernels, whose waves have no other LDS work to hide
// the latency behind).
template <bool PX = false> __device__ __forceinline__ float q6k_dot(uint4 (&c)[13], uint32_t dbits, dfloat *x)
{
	// inputs of half step hs = 2 st + half: x[128n + l + 4hw + 64 half + {0, 32} ..]
	auto xat = [&](int hs) {
		const int st = hs >> 1, half = hs & 1;
		return x + 128 * (st >> 3) + 8 * ((st >> 1) & 3) + 4 * (st & 1) + 64 * half;
	};
	vf4 pa, pc;
	if constexpr (PX) {
		pa = *(dfloat4 *)xat(0);
		pc = *(dfloat4 *)(xat(0) + 32);
	}
	const float d = half_bits_to_float(dbits);
	uint4 sc4 = c[12];
	auto sc = [&](int j) { return (float)(int8_t)((dword_of(sc4, j >> 2) >> (8 * (j & 3))) & 0xffu); };
	float a0[8], a1[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		a0[l] = a1[l] = 0.0f;
#pragma unroll
	for (int st = 0; st < 16; st++) {
		const int qt = st >> 2, n = st >> 3, l = 8 * ((st >> 1) & 3), hw = st & 1;
		const int hl = qt & 1, is = (l >= 16) ? 1 : 0;
		if ((st & 3) == 0) {
			// one quarter at a time
			acc_fence(a0, a1);
			if constexpr (!PX)
				asm volatile("" : "+v"(x));
			pin(sc4);
			pin(c[4 * n + hl]);
			pin(c[4 * n + 2 + hl]);
			pin(c[8 + 2 * n + hl]);
		}
		// quarter qt = (n, hl): ql chunks 4n + hl (low nibbles) and 4n + 2 + hl
		// (high nibbles), qh chunk 8 + 2n + hl
		const uint4 &C0 = c[4 * n + hl], &C1 = c[4 * n + 2 + hl], &C2 = c[8 + 2 * n + hl];
		const float W0 = d * sc(8 * n + is + 0), W1 = d * sc(8 * n + is + 2);
		const float W2 = d * sc(8 * n + is + 4), W3 = d * sc(8 * n + is + 6);
		const int dw = ((l & 8) >> 2) + hw;
		const uint32_t L = dword_of(C0, dw), L2 = dword_of(C1, dw), H = dword_of(C2, dw);
		// bytes of q - 32
		const uint32_t q1 = q6_codes(L, 0, H, 0), q2 = q6_codes(L2, 0, H, 2);
		const uint32_t q3 = q6_codes(L, 4, H, 4), q4 = q6_codes(L2, 4, H, 6);
		dfloat *xb = x + 128 * n + l + 4 * hw;
#pragma unroll
		for (int half = 0; half < 2; half++) {
			uint32_t qa = half ? q3 : q1, qb = half ? q4 : q2;
			asm volatile("" : "+v"(qa), "+v"(qb)); // byte-parallel codes (one conversion each)
			const float Wa = half ? W2 : W0, Wb = half ? W3 : W1;
			vf4 xa, xc;
			if constexpr (PX) {
				xa = pa;
				xc = pc;
				const int hs = 2 * st + half;
				if (hs + 1 < 32) {
					pa = *(dfloat4 *)xat(hs + 1);
					pc = *(dfloat4 *)(xat(hs + 1) + 32);
				}
			} else {
				xa = *(dfloat4 *)(xb + 64 * half);
				xc = *(dfloat4 *)(xb + 64 * half + 32);
			}
			const float xav[4] = {xa.x, xa.y, xa.z, xa.w}, xcv[4] = {xc.x, xc.y, xc.z, xc.w};
#pragma unroll
			for (int i = 0; i < 4; i++) {
				const int m = 4 * hw + i;
				const float fa = sbyte_f(qa, i), fb = sbyte_f(qb, i);
				a0[m] = __builtin_fmaf(Wa, fa * xav[i], a0[m]);
				a1[m] = __builtin_fmaf(Wb, fb * xcv[i], a1[m]);
			}
		}
	}
	float v[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		v[l] = a0[l] + a1[l];
	return hsum8(v);
}

typedef const uint4 __attribute__((address_space(1))) g4;

// One (row, block) of a quantised tensor held in registers: `blk` = the
// row's 16-byte slot in chunk 0 of its panel's block column (chunk c at
// +1024 c), `dp` (Q6_K) = the row's fp16 d.  load() issues every load of the
// block; dot() waits for them as it goes.
template <int TYPE> struct RowBlock;
template <> struct RowBlock<TIE_GGML_Q4_K> {
	uint4 c[9];
	__device__ __forceinline__ void load(const uint8_t *blk, const uint8_t *)
	{
#pragma unroll
		for (int i = 0; i < 9; i++)
			c[i] = *(const uint4 *)(g4 *)(blk + 1024 * i);
	}
	template <bool PX = false> __device__ __forceinline__ float dot(dfloat *x) { return q4k_dot(c, x); }
};
template <> struct RowBlock<TIE_GGML_Q6_K> {
	uint4 c[13];
	uint32_t db;
	__device__ __forceinline__ void load(const uint8_t *blk, const uint8_t *dp)
	{
#pragma unroll
		for (int i = 0; i < 13; i++)
			c[i] = *(const uint4 *)(g4 *)(blk + 1024 * i);
		db = *(const uint16_t *)dp;
	}
	template <bool PX = false> __device__ __forceinline__ float dot(dfloat *x) { return q6k_dot<PX>(c, db, x); }
};


// ---- block dots by two adjacent lanes (lanes 2i and 2i + 1 of a wave, both
// active).  Each lane loads only the code words of its half of the steps,
// keeps the accumulators those steps update (a step's accumulators belong
// to one half), and lane 2i ends with the block's dot: TIE's FMAs in TIE's
// order per accumulator, then hsum_f32_avx2's tree.  Half the registers and
// half the dependent work of RowBlock per lane.
typedef const uint2 __attribute__((address_space(1))) g2;
typedef const uint32_t __attribute__((address_space(1))) g1;

__device__ __forceinline__ void pin2(uint2 &v)
{
	asm volatile("" : "+v"(v.x), "+v"(v.y));
}

template <int TYPE> struct PairBlock;

// Q4_K (q4k_dot): lane p takes dwords 2p, 2p + 1 of every code chunk, the
// steps h = 2p, 2p + 1, whose accumulators 4h + i are a0 (p = 0) or a1 (p =
// 1); v[l] = a0[l] + a1[l] on lane 0 with a1 moved over from lane 1.
template <> struct PairBlock<TIE_GGML_Q4_K> {
	uint4 s;    // chunk 0: d, dmin, scales
	uint2 q[8]; // dwords 2p, 2p + 1 of code chunks 1..8
	__device__ __forceinline__ void load(const uint8_t *blk, const uint8_t *, int p)
	{
		s = *(const uint4 *)(g4 *)blk;
#pragma unroll
		for (int i = 0; i < 8; i++)
			q[i] = *(const uint2 *)(g2 *)(blk + 1024 * (1 + i) + 8 * p);
	}
	template <bool PX = false> __device__ __forceinline__ float dot(dfloat *x, int p)
	{
		const float d = half_bits_to_float(s.x & 0xffffu);
		const float dmin = half_bits_to_float(s.x >> 16);
		float a[8];
#pragma unroll
		for (int l = 0; l < 8; l++)
			a[l] = 0.0f;
		dfloat *xp = x + 8 * p;
#pragma unroll
		for (int g = 0; g < 4; g++) {
			asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]),
					  "+v"(a[7]));
			asm volatile("" : "+v"(xp));
			pin2(q[2 * g]);
			pin2(q[2 * g + 1]);
			float D1, M1, D2, M2;
			q4k_scale(s, 2 * g, d, dmin, D1, M1);
			q4k_scale(s, 2 * g + 1, d, dmin, D2, M2);
#pragma unroll
			for (int o = 0; o < 2; o++) {
#pragma unroll
				for (int hh = 0; hh < 2; hh++) {
					const uint32_t w = hh ? q[2 * g + o].y : q[2 * g + o].x;
					uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
					asm volatile("" : "+v"(lo), "+v"(hi));
					dfloat *xb = xp + 64 * g + 16 * o + 4 * hh; // step h = 2p + hh
					const vf4 xl = *(dfloat4 *)xb, xh = *(dfloat4 *)(xb + 32);
					const float xlv[4] = {xl.x, xl.y, xl.z, xl.w}, xhv[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
					for (int i = 0; i < 4; i++) {
						const float wl = __builtin_fmaf(byte_f(lo, i), D1, M1);
						const float wh = __builtin_fmaf(byte_f(hi, i), D2, M2);
						float &A = a[4 * hh + i];
						A = __builtin_fmaf(xlv[i], wl, A);
						A = __builtin_fmaf(xhv[i], wh, A);
					}
				}
			}
		}
		float v[8];
#pragma unroll
		for (int l = 0; l < 8; l++)
			v[l] = a[l] + dppf<DPP_SHL1>(a[l]);
		return hsum8(v);
	}
};

// Q6_K (q6k_dot): lane p takes the steps hw = p (dwords p and p + 2 of the
// ql / qh chunks), whose accumulators are 4p + i of a0 and of a1, so v[4p +
// i] = a0 + a1 is local; hsum_f32_avx2's first level v[i] + v[i + 4] takes
// lane 1's four on lane 0.  PX: each half step's inputs read one half step
// ahead.
template <> struct PairBlock<TIE_GGML_Q6_K> {
	uint32_t ql[8][2]; // dwords p, p + 2 of the ql chunks
	uint32_t qh[4][2]; // of the qh chunks
	uint4 sc4;         // the int8 scales
	uint32_t db;       // fp16 d
	__device__ __forceinline__ void load(const uint8_t *blk, const uint8_t *dp, int p)
	{
#pragma unroll
		for (int c = 0; c < 8; c++) {
			ql[c][0] = *(const uint32_t *)(g1 *)(blk + 1024 * c + 4 * p);
			ql[c][1] = *(const uint32_t *)(g1 *)(blk + 1024 * c + 8 + 4 * p);
		}
#pragma unroll
		for (int c = 0; c < 4; c++) {
			qh[c][0] = *(const uint32_t *)(g1 *)(blk + 1024 * (8 + c) + 4 * p);
			qh[c][1] = *(const uint32_t *)(g1 *)(blk + 1024 * (8 + c) + 8 + 4 * p);
		}
		sc4 = *(const uint4 *)(g4 *)(blk + 1024 * 12);
		db = *(const uint16_t *)dp;
	}
	template <bool PX = false> __device__ __forceinline__ float dot(dfloat *x, int p)
	{
		dfloat *xp = x + 4 * p;
		// inputs of half step hs = 2 s + half of this lane's steps s
		auto xat = [&](int hs) {
			const int st = hs >> 1, half = hs & 1;
			return xp + 128 * (st >> 2) + 8 * (st & 3) + 64 * half;
		};
		vf4 pa, pc;
		if constexpr (PX) {
			pa = *(dfloat4 *)xat(0);
			pc = *(dfloat4 *)(xat(0) + 32);
		}
		const float d = half_bits_to_float(db);
		auto sc = [&](int j) { return (float)(int8_t)((dword_of(sc4, j >> 2) >> (8 * (j & 3))) & 0xffu); };
		float a0[4], a1[4];
#pragma unroll
		for (int i = 0; i < 4; i++)
			a0[i] = a1[i] = 0.0f;
#pragma unroll
		for (int st = 0; st < 8; st++) {
			// this lane's step st = q6k_dot's step 2 st + p
			const int qt = st >> 1, n = st >> 2, l = 8 * (st & 3), hl = qt & 1, is = (l >= 16) ? 1 : 0;
			const int w = st & 1; // dword p (0) or p + 2 (1)
			if ((st & 1) == 0) {
				asm volatile("" : "+v"(a0[0]), "+v"(a0[1]), "+v"(a0[2]), "+v"(a0[3]), "+v"(a1[0]), "+v"(a1[1]),
						  "+v"(a1[2]), "+v"(a1[3]));
				if constexpr (!PX)
					asm volatile("" : "+v"(xp));
				asm volatile("" : "+v"(sc4.x), "+v"(sc4.y), "+v"(sc4.z), "+v"(sc4.w));
				asm volatile("" : "+v"(ql[4 * n + hl][0]), "+v"(ql[4 * n + hl][1]), "+v"(ql[4 * n + 2 + hl][0]),
						  "+v"(ql[4 * n + 2 + hl][1]), "+v"(qh[2 * n + hl][0]), "+v"(qh[2 * n + hl][1]));
			}
			const float W0 = d * sc(8 * n + is + 0), W1 = d * sc(8 * n + is + 2);
			const float W2 = d * sc(8 * n + is + 4), W3 = d * sc(8 * n + is + 6);
			const uint32_t L = ql[4 * n + hl][w], L2 = ql[4 * n + 2 + hl][w], H = qh[2 * n + hl][w];
			const uint32_t q1 = q6_codes(L, 0, H, 0), q2 = q6_codes(L2, 0, H, 2);
			const uint32_t q3 = q6_codes(L, 4, H, 4), q4 = q6_codes(L2, 4, H, 6);
#pragma unroll
			for (int half = 0; half < 2; half++) {
				uint32_t qa = half ? q3 : q1, qb = half ? q4 : q2;
				asm volatile("" : "+v"(qa), "+v"(qb));
				const float Wa = half ? W2 : W0, Wb = half ? W3 : W1;
				vf4 xa, xc;
				if constexpr (PX) {
					xa = pa;
					xc = pc;
					const int hs = 2 * st + half;
					if (hs + 1 < 16) {
						pa = *(dfloat4 *)xat(hs + 1);
						pc = *(dfloat4 *)(xat(hs + 1) + 32);
					}
				} else {
					xa = *(dfloat4 *)xat(2 * st + half);
					xc = *(dfloat4 *)(xat(2 * st + half) + 32);
				}
				const float xav[4] = {xa.x, xa.y, xa.z, xa.w}, xcv[4] = {xc.x, xc.y, xc.z, xc.w};
#pragma unroll
				for (int i = 0; i < 4; i++) {
					const float fa = sbyte_f(qa, i), fb = sbyte_f(qb, i);
					a0[i] = __builtin_fmaf(Wa, fa * xav[i], a0[i]);
					a1[i] = __builtin_fmaf(Wb, fb * xcv[i], a1[i]);
				}
			}
		}
		float v[4];
#pragma unroll
		for (int i = 0; i < 4; i++)
			v[i] = a0[i] + a1[i];
		float s4[4];
#pragma unroll
		for (int i = 0; i < 4; i++)
			s4[i] = v[i] + dppf<DPP_SHL1>(v[i]); // lane 0: v[i] + v[i + 4]
		return (s4[0] + s4[1]) + (s4[2] + s4[3]);
	}
};

// One (row, block) dot per lane (RowBlock) or per pair of lanes (PairBlock)
// behind one interface; hp = the lane's half (0 without pairs).
template <int TYPE, bool PAIR> struct LaneBlock : PairBlock<TYPE> {
};
template <int TYPE> struct LaneBlock<TYPE, false> {
	RowBlock<TYPE> rb;
	__device__ __forceinline__ void load(const uint8_t *blk, const uint8_t *dp, int) { rb.load(blk, dp); }
	template <bool PX = false> __device__ __forceinline__ float dot(dfloat *x, int)
	{
		return rb.template dot<PX>(x);
	}
};

// the row's fp16 d in a Q6_K panel (the d plane after the 13 chunks)
__device__ __forceinline__ const uint8_t *q6k_d_of(const uint8_t *blk, int row)
{
	return blk + Q6K_CHUNKS * 1024 - 14 * (row & 63);
}

// The dot of one (row, block) with the input segment x (all loads issued
// before any use).
template <int TYPE> __device__ __forceinline__ float row_block_dot(const uint8_t *blk, const uint8_t *dp, dfloat *x)
{
	RowBlock<TYPE> rb;
	rb.load(blk, dp);
	return rb.dot(x);
}

// address of row `row`, block column b of expert e (panel layout)
__device__ __forceinline__ const uint8_t *panel_slot(const uint8_t *base, size_t expert_bytes, int e, int row, int b,
						     int nb, size_t pbytes)
{
	return base + (size_t)e * expert_bytes + ((size_t)(row >> 6) * nb + b) * pbytes + (row & 63) * 16;
}

struct DecodeArgs {
	const uint8_t *w[3];   // gate, up, down (panel layout)
	size_t expert_bytes[3];
	int d, F, E, k;
	int R;                 // rows per workgroup (a power of two <= 64)
	const float *x;        // [T][d]
	const float *logits;   // [T][E] (inline routing)
	int32_t *topk_idx;     // [T][k]
	float *topk_w;         // [T][k]
	float *h;              // [list entry][k][F] SwiGLU outputs
	float *out;            // [T][d]
	const float *res;      // [T][d] or null: out = res + block
	const float *silu;
	const int32_t *list;   // tokens to run (null: token 0 only)
	const int32_t *count;  // number of list entries (device)
	int routing;
	const float *pbias;
};

__device__ __forceinline__ int list_count(const DecodeArgs &a)
{
	return a.list ? __builtin_amdgcn_readfirstlane(*a.count) : 1;
}

__device__ __forceinline__ int list_token(const DecodeArgs &a, int li)
{
	return a.list ? __builtin_amdgcn_readfirstlane(a.list[li]) : 0;
}

// Dynamic LDS: x [nb][XSEG] | part [2 nb][R] | (INLINE) selection
// Row sums of the gate/up partial dots part[(m nb + b) R + r] (m = 0 gate,
// 1 up): s = 0 + p_0 + p_1 + ... in block order (math_avx2.c:762-766), one
// thread per (matrix, row), into part[m R + r] (after a barrier).
__device__ __forceinline__ void row_sums(float *part, int nb, int R)
{
	float s = 0.0f;
	const int t = threadIdx.x;
	if (t < 2 * R) {
		const int m = t / R, r = t - m * R;
#pragma unroll 8
		for (int b = 0; b < nb; b++)
			s = s + part[(m * nb + b) * R + r];
	}
	__syncthreads();
	if (t < 2 * R)
		part[t] = s;
	__syncthreads();
}

// The combine of R rows from the down partial dots part[(j nb + b) R + r],
// one thread per row: y_j = serial block sum per slot, out = fma(g_j, y_j,
// .) in slot order from +0 (model_qwen3.c:459-467; slots without an expert
// add nothing), [res +].  The partial dots of several slots are read ahead
// of their sums (the loop is unrolled), so one LDS latency is exposed per
// few slots, not one per read; no barrier.
__device__ __forceinline__ void combine_rows(const float *part, int nb, int k, int R, const int32_t *sel_idx,
					     const float *sel_w, float *out, const float *res)
{
	const int t = threadIdx.x;
	if (t >= R)
		return;
	float acc = 0.0f;
#pragma unroll 4
	for (int j = 0; j < k; j++) {
		const float *pj = part + (size_t)j * nb * R + t;
		float y = 0.0f;
#pragma unroll 4
		for (int b = 0; b < nb; b++)
			y = y + pj[b * R];
		if (sel_idx[j] >= 0)
			acc = __builtin_fmaf(sel_w[j], y, acc);
	}
	out[t] = res ? res[t] + acc : acc;
}

template <int TG, int TU, bool INLINE>
__global__ __launch_bounds__(DEC_MAX_THREADS) void decode_gu_kernel(DecodeArgs a)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	__shared__ int32_t sel_idx[MAX_K];
	__shared__ float sel_w[MAX_K];
	__shared__ uint64_t etab[32];
	__shared__ float slg[INLINE_E]; // the token's logits (E <= INLINE_E with inline routing)
	const int R = a.R, j = blockIdx.y;
	const int nb = a.d / QK;
	float *xs = dl;
	float *part = dl + nb * XSEG;
	const int tid = threadIdx.x;
	const int ntask = 2 * nb;
	const int n = list_count(a);
	for (int li = blockIdx.z; li < n; li += gridDim.z) {
		const int t = list_token(a, li);
		// x of the token (and its logits) -> LDS in one round trip
		copy_in<4>(reinterpret_cast<const float4 *>(a.x + (size_t)t * a.d), a.d / 4, [&](int q, float4 v) {
			const int f = 4 * q;
			*reinterpret_cast<float4 *>(xs + (f / QK) * XSEG + (f % QK)) = v;
		});
		int e;
		if constexpr (INLINE) {
			// the token's selection from its logits (one wave), published
			// by workgroup (0, 0) for the down kernel
			if (tid < 32) {
				const uint64_t tab[32] = TIE_EXP2_TABLE;
				etab[tid] = tab[tid];
			}
			for (int i = tid; i < a.E; i += blockDim.x)
				slg[i] = a.logits[(size_t)t * a.E + i];
			__syncthreads();
			if (tid < 64)
				topk_softmax_wave<2>(slg, a.E, a.k, etab, sel_idx, sel_w, a.routing, a.pbias);
			__syncthreads();
			if (blockIdx.x == 0 && j == 0 && tid < a.k) {
				a.topk_idx[(size_t)t * a.k + tid] = sel_idx[tid];
				a.topk_w[(size_t)t * a.k + tid] = sel_w[tid];
			}
			e = sel_idx[j];
		} else {
			e = __builtin_amdgcn_readfirstlane(a.topk_idx[(size_t)t * a.k + j]);
			__syncthreads();
		}
		if (e < 0) // slot without an expert: its h is never read
			continue;
		const int r0 = blockIdx.x * R;
		for (int u = tid; u < ntask * R; u += blockDim.x) {
			const int r = u & (R - 1), task = u / R;
			const int mat = task >= nb ? 1 : 0, b = task - mat * nb;
			const uint8_t *blk = panel_slot(a.w[mat], a.expert_bytes[mat], e, r0 + r, b, nb,
							panel_bytes(mat ? TU : TG));
			float v;
			if (mat == 0)
				v = row_block_dot<TG>(blk, q6k_d_of(blk, r0 + r), (dfloat *)(xs + b * XSEG));
			else
				v = row_block_dot<TU>(blk, q6k_d_of(blk, r0 + r), (dfloat *)(xs + b * XSEG));
			part[task * R + r] = v;
		}
		__syncthreads();
		// serial sums over the blocks (math_avx2.c:762-766), SwiGLU
		row_sums(part, nb, R);
		if (tid < R)
			a.h[((size_t)li * a.k + j) * a.F + r0 + tid] = tie_swiglu(part[tid], part[R + tid], a.silu);
		__syncthreads();
	}
}

// Dynamic LDS: h [k][nb][XSEG] | part [k nb][R]
template <int TD> __global__ __launch_bounds__(DEC_MAX_THREADS) void decode_down_kernel(DecodeArgs a)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	__shared__ int32_t sel_idx[MAX_K];
	__shared__ float sel_w[MAX_K];
	const int R = a.R, k = a.k;
	const int nb = a.F / QK;
	float *hs = dl;
	float *part = dl + (size_t)k * nb * XSEG;
	const int tid = threadIdx.x;
	const int ntask = k * nb;
	const int n = list_count(a);
	const int r0 = blockIdx.x * R;
	for (int li = blockIdx.z; li < n; li += gridDim.z) {
		const int t = list_token(a, li);
		if (tid < k) {
			sel_idx[tid] = a.topk_idx[(size_t)t * k + tid];
			sel_w[tid] = a.topk_w[(size_t)t * k + tid];
		}
		// the k h vectors -> LDS (independent of the selection), one round trip
		copy_in<8>(reinterpret_cast<const float4 *>(a.h + (size_t)li * k * a.F), k * a.F / 4, [&](int q, float4 v) {
			const int f = 4 * q; // = j F + b QK + m
			*reinterpret_cast<float4 *>(hs + (f / QK) * XSEG + (f % QK)) = v;
		});
		__syncthreads();
		for (int u = tid; u < ntask * R; u += blockDim.x) {
			const int r = u & (R - 1), task = u / R;
			const int j = task / nb, b = task - j * nb;
			const int e = sel_idx[j];
			float v = 0.0f;
			if (e >= 0) {
				const uint8_t *blk = panel_slot(a.w[2], a.expert_bytes[2], e, r0 + r, b, nb, panel_bytes(TD));
				v = row_block_dot<TD>(blk, q6k_d_of(blk, r0 + r), (dfloat *)(hs + (size_t)task * XSEG));
			}
			part[task * R + r] = v;
		}
		__syncthreads();
		combine_rows(part, nb, k, R, sel_idx, sel_w, a.out + (size_t)t * a.d + r0, a.res ? a.res + (size_t)t * a.d + r0 : nullptr);
		__syncthreads();
	}
}

// ------------------------------------------------------------ one launch
// T = 1 in a single launch.  Workgroups take one of three roles by index,
// in dependency order (the dispatcher starts workgroups in index order, so a
// workgroup only ever waits for workgroups started before it):
//
//   [0, nr)          router: rpr expert rows each, TIE's 8 lane chains and
//                    hsum tree (as router_small_kernel).
//   [nr, nr + ng)    gate/up: (slot j, rg rows of F): x staged while the
//                    router runs, the logits read back, the token's
//                    selection made in the prologue (as decode_gu_kernel),
//                    h = silu_tab(gate) * up published.
//   [nr + ng, ...)   down + combine: (rd rows of d): the selection made
//                    again from the logits, every weight block of the
//                    workgroup's rows loaded into registers BEFORE the wait
//                    for h, then the dots and the combine (as
//                    decode_down_kernel).
//
// Every value handed between workgroups (the E logits, the k F values of
// h) travels as one 64-bit word {seq, value bits}, written and read with
// agent-scope relaxed atomics (sc1: coherent across the XCDs' L2s with no
// cache write-back, invalidate or separate flag); seq (one per call) tells
// a word of this call from one left by an earlier call.  The waits are
// bounded (spin polls): a wait that gives up produces NaN outputs instead
// of hanging, and sets the call's status word, which the host reads back
// (tie_hip_stream_status; the synchronous entry points return the error).

__device__ __forceinline__ unsigned long long ld_word(const unsigned long long *p)
{
	return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long wait_word64(const unsigned long long *p, uint32_t seq, int spin, int &bad)
{
	for (int i = 0; i < spin; i++) {
		const unsigned long long v = ld_word(p);
		if ((uint32_t)(v >> 32) == seq)
			return v;
		__builtin_amdgcn_s_sleep(1);
	}
	bad = 1;
	return 0x7fc00000ull; // NaN
}

struct OneArgs {
	DecodeArgs a;
	const float *router;      // [E][d] F32 rows
	const float *bias;        // [E] or null
	unsigned long long *lg;   // [ONE_LG_COPIES][E] {seq, logit}, copies lg_copy words apart
	unsigned long long *hw;   // [ONE_H_COPIES][k][F] {seq, h}, copies hw_copy words apart
	size_t lg_copy, hw_copy;
	uint32_t seq;             // the stamp this call writes
	uint32_t wseq;            // the stamp its waits look for (seq; another value only from the debug hook)
	int spin;                 // polls before a wait gives up
	int32_t *status;          // set to 1 when a wait gave up
	int nr, ng;               // router, gate/up workgroups
	int rpr, rg, rd;          // rows per router, gate/up, down workgroup
};

#ifdef TIE_ONE_TRACE
// diagnostic timeline of the one-launch decode (s_memrealtime, 100 MHz):
// [2i] earliest, [2i+1] latest time of event i over the workgroups
constexpr int ONE_TRACE_WG = 8192;
__device__ unsigned long long g_one_trace[ONE_TRACE_WG][8]; // role + 1, stamps, (down) core clock at start / end
__device__ __forceinline__ void one_mark(int i, unsigned long long t)
{
	if (blockIdx.x < ONE_TRACE_WG) {
		g_one_trace[blockIdx.x][0] = 1 + (i >= 6 ? 2 : i >= 3 ? 1 : 0);
		g_one_trace[blockIdx.x][1 + (i >= 6 ? i - 6 : i >= 3 ? i - 3 : i)] = t;
	}
}
#define ONE_T(v) const unsigned long long v = __builtin_amdgcn_s_memrealtime()
#else
#define ONE_T(v)
#endif
// The token's logits (published by the router workgroups), read back by
// thread e, then its selection -> sel_idx / sel_w.  Ends with a barrier.
__device__ __forceinline__ void one_select(const OneArgs &o, uint64_t *etab, int32_t *sel_idx, float *sel_w, int *sbad,
					   RankScratch *rs, bool weights)
{
	const int tid = threadIdx.x;
	if (tid < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		etab[tid] = tab[tid];
	}
	__syncthreads();
	if (tid < o.a.E) {
		int bad = 0;
		const unsigned long long *lg = o.lg + (blockIdx.x % ONE_LG_COPIES) * o.lg_copy;
		const float v = __uint_as_float((uint32_t)wait_word64(lg + tid, o.wseq, o.spin, bad));
		if (bad)
			*sbad = 1;
		rank_key(v, tid, o.a.routing, o.a.pbias, etab, *rs);
	}
#ifdef TIE_ONE_TRACE
	__syncthreads();
	if (tid == 0 && blockIdx.x < ONE_TRACE_WG)
		g_one_trace[blockIdx.x][5] = __builtin_amdgcn_s_memrealtime();
#endif
	topk_rank_block(o.a.E, o.a.k, etab, sel_idx, sel_w, o.a.routing, *rs, weights);
}

template <int TG, int TU, int TD, bool PAIR>
__global__ __launch_bounds__(DEC_MAX_THREADS, PAIR ? ONE_PAIR_WAVES : 4) void decode_one_kernel(const OneArgs o_arg)
{
	constexpr int LP = PAIR ? 2 : 1; // lanes per (row, block) dot
	ONE_T(t_start);
	extern __shared__ __attribute__((aligned(16))) float dl[];
	__shared__ int32_t sel_idx[MAX_K];
	__shared__ float sel_w[MAX_K];
	__shared__ uint64_t etab[32];
	__shared__ RankScratch rsc;
	__shared__ int sbad;
	const int tid = threadIdx.x, b = blockIdx.x;
	const OneArgs &o = o_arg;
	const DecodeArgs &a = o.a;
	const int d = a.d;
	if (tid == 0)
		sbad = 0;
	if (b < o.nr) {
		// ---- router rows e0 .. e0 + ne - 1
		const int e0 = b * o.rpr, ne = min(o.rpr, a.E - e0);
		const int lmf = lane_major_floats(d), st = lane_major_stride(d), n4 = d / 4;
		// x and the rows -> LDS lane-major, all loads of a thread in flight at once
		for (int base = tid; base < (1 + ne) * n4; base += 8 * (int)blockDim.x) {
			float4 v[8];
#pragma unroll
			for (int i = 0; i < 8; i++) {
				const int q = base + i * (int)blockDim.x;
				const int r = q / n4, c = q - r * n4;
				const float *src = r == 0 ? a.x : o.router + (size_t)(e0 + r - 1) * d;
				v[i] = q < (1 + ne) * n4 ? reinterpret_cast<const float4 *>(src)[c] : make_float4(0, 0, 0, 0);
			}
#pragma unroll
			for (int i = 0; i < 8; i++) {
				const int q = base + i * (int)blockDim.x;
				if (q < (1 + ne) * n4) {
					const int r = q / n4, f = 4 * (q - r * n4), l = f & 7, ii = f >> 3;
					float *dst = dl + r * lmf;
					dst[(l + 0) * st + ii] = v[i].x;
					dst[(l + 1) * st + ii] = v[i].y;
					dst[(l + 2) * st + ii] = v[i].z;
					dst[(l + 3) * st + ii] = v[i].w;
				}
			}
		}
		__syncthreads();
		ONE_T(t_staged);
		if (tid < 8 * ne) {
			const int r = tid >> 3, l = tid & 7;
			const float s = hsum8_lanes(lane_chain(dl, dl + (1 + r) * lmf, d, l));
			if (l == 0) {
				const int e = e0 + r;
				const float v = o.bias ? s + o.bias[e] : s;
				const unsigned long long w = ((unsigned long long)o.seq << 32) | __float_as_uint(v);
#pragma unroll
				for (int c = 0; c < ONE_LG_COPIES; c++)
					__hip_atomic_store(o.lg + c * o.lg_copy + e, w, __ATOMIC_RELAXED,
							   __HIP_MEMORY_SCOPE_AGENT);
			}
		}
#ifdef TIE_ONE_TRACE
		if (tid == 0) {
			ONE_T(t_end);
			one_mark(0, t_start);
			one_mark(1, t_staged);
			one_mark(2, t_end);
		}
#endif
		return;
	}
	if (b < o.nr + o.ng) {
		// ---- gate/up: slot j, rows r0 .. r0 + rg - 1 of F
		const int gb = b - o.nr, nxg = a.F / o.rg, R = o.rg;
		const int j = gb / nxg, r0 = (gb - j * nxg) * R;
		const int nb = d / QK;
		float *xs = dl;
		float *part = dl + nb * XSEG;
		copy_in<4>(reinterpret_cast<const float4 *>(a.x), d / 4, [&](int q, float4 v) {
			const int f = 4 * q;
			*reinterpret_cast<float4 *>(xs + (f / QK) * XSEG + (f % QK)) = v;
		});
		// the experts only: their gate weights (topk_w, by the first
		// gate/up workgroup) wait until its h is out
		one_select(o, etab, sel_idx, sel_w, &sbad, &rsc, false);
		ONE_T(t_sel);
		const int e = sel_idx[j];
		float hv = 0.0f; // a slot without an expert: its h is never used
		if (e >= 0) {
			// lanes (task, row[, half]): LP lanes per (row, block)
			for (int u2 = tid; u2 < LP * 2 * nb * R; u2 += blockDim.x) {
				const int hp = u2 & (LP - 1), u = u2 / LP;
				const int task = u / R, r = u - task * R;
				const int mat = task >= nb ? 1 : 0, bb = task - mat * nb;
				const uint8_t *blk = panel_slot(a.w[mat], a.expert_bytes[mat], e, r0 + r, bb, nb,
								panel_bytes(mat ? TU : TG));
				float v;
				if (mat == 0) {
					LaneBlock<TG, PAIR> pb;
					pb.load(blk, q6k_d_of(blk, r0 + r), hp);
					v = pb.dot((dfloat *)(xs + bb * XSEG), hp);
				} else {
					LaneBlock<TU, PAIR> pb;
					pb.load(blk, q6k_d_of(blk, r0 + r), hp);
					v = pb.dot((dfloat *)(xs + bb * XSEG), hp);
				}
				if (hp == 0)
					part[task * R + r] = v;
			}
			__syncthreads();
			row_sums(part, nb, R);
			if (tid < R)
				hv = sbad ? __builtin_nanf("") : tie_swiglu(part[tid], part[R + tid], a.silu);
		}
		if (tid < R) {
			const unsigned long long w = ((unsigned long long)o.seq << 32) | __float_as_uint(hv);
#pragma unroll
			for (int c = 0; c < ONE_H_COPIES; c++)
				__hip_atomic_store(o.hw + c * o.hw_copy + (size_t)j * a.F + r0 + tid, w, __ATOMIC_RELAXED,
						   __HIP_MEMORY_SCOPE_AGENT);
		}
		if (sbad && tid == 0)
			__hip_atomic_store(o.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		if (gb == 0) {
			topk_rank_weights(a.k, etab, sel_idx, sel_w, a.routing, rsc);
			if (tid < a.k) {
				a.topk_idx[tid] = sel_idx[tid];
				a.topk_w[tid] = sel_w[tid];
			}
		}
#ifdef TIE_ONE_TRACE
		if (tid == 0) {
			ONE_T(t_end);
			one_mark(3, t_start);
			one_mark(4, t_sel);
			one_mark(5, t_end);
		}
#endif
		return;
	}
	// ---- down + combine: rows r0 .. r0 + rd - 1 of d; lane (task, row): the
	// block dot of (row, slot j, block b), task = j nb + b
	const int R = o.rd, k = a.k, nb = a.F / QK;
	const int r0 = (b - o.nr - o.ng) * R;
#ifdef TIE_ONE_TRACE
	const unsigned long long c_start = __builtin_amdgcn_s_memtime();
#endif
	float *hs = dl;                           // [k nb][XSEG]
	float *part = dl + (size_t)k * nb * XSEG; // [k nb][R]
	one_select(o, etab, sel_idx, sel_w, &sbad, &rsc, false);
	ONE_T(t_sel);
	// lanes (task, row[, half]): LP lanes per (row, block)
	const int ntask = k * nb, hp = tid & (LP - 1);
	const int task = (tid / LP) / R, r = (tid / LP) - task * R;
	const bool live = task < ntask;
	const int jj = live ? task / nb : 0, bb = live ? task - jj * nb : 0;
	const int e = live ? sel_idx[jj] : -1;
	LaneBlock<TD, PAIR> rb;
	{
		// the weights before the wait for h (unconditional: a lane without
		// an expert reads expert 0's block and never uses it; a conditional
		// load would have the compiler wait for it at once)
		const int rr = live ? r0 + r : r0;
		const uint8_t *blk = panel_slot(a.w[2], a.expert_bytes[2], e >= 0 ? e : 0, rr, bb, nb, panel_bytes(TD));
		rb.load(blk, q6k_d_of(blk, rr), hp);
	}
	// the gate weights while those loads are in flight
	topk_rank_weights(k, etab, sel_idx, sel_w, a.routing, rsc);

	// h (k F words of this call) -> LDS, 8 words of a thread polled at
	// once, the ones not yet stamped again until all are
	{
		const int nw = k * a.F;
		const unsigned long long *hw = o.hw + (blockIdx.x % ONE_H_COPIES) * o.hw_copy;
		int bad = 0;
		for (int base = tid; base < nw; base += 8 * (int)blockDim.x) {
			unsigned long long v[8];
			uint32_t pend = 0;
#pragma unroll
			for (int i = 0; i < 8; i++)
				if (base + i * (int)blockDim.x < nw)
					pend |= 1u << i;
			int it = 0;
			while (pend) {
#pragma unroll
				for (int i = 0; i < 8; i++)
					if (pend & (1u << i))
						v[i] = ld_word(hw + base + i * (int)blockDim.x);
#pragma unroll
				for (int i = 0; i < 8; i++)
					if ((pend & (1u << i)) && (uint32_t)(v[i] >> 32) == o.wseq) {
						pend &= ~(1u << i);
						const int f = base + i * (int)blockDim.x; // = (j nb + b) QK + m
						hs[(f / QK) * XSEG + f % QK] = __uint_as_float((uint32_t)v[i]);
					}
				if (pend && ++it >= o.spin) {
					bad = 1;
					break;
				}
				if (pend)
					__builtin_amdgcn_s_sleep(1);
			}
		}
		if (bad)
			sbad = 1;
	}
	__syncthreads();
	ONE_T(t_h);
	if (live) {
		const float v = e >= 0 ? rb.template dot<true>((dfloat *)(hs + (size_t)task * XSEG), hp) : 0.0f;
		if (hp == 0)
			part[task * R + r] = v;
	}
	__syncthreads();
#ifdef TIE_ONE_TRACE
	if (tid == 0 && blockIdx.x < ONE_TRACE_WG)
		g_one_trace[blockIdx.x][5] = __builtin_amdgcn_s_memrealtime(); // the down dots done
#endif
	float *outp = a.out + r0;
	combine_rows(part, nb, k, R, sel_idx, sel_w, outp, a.res ? a.res + r0 : nullptr);
	if (sbad && tid < R)
		outp[tid] = __builtin_nanf("");
	if (sbad && tid == 0)
		__hip_atomic_store(o.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef TIE_ONE_TRACE
	if (tid == 0) {
		ONE_T(t_end);
		one_mark(6, t_start);
		g_one_trace[blockIdx.x][6] = c_start;
		g_one_trace[blockIdx.x][7] = __builtin_amdgcn_s_memtime();
		one_mark(7, t_sel);
		one_mark(8, t_h);
		one_mark(9, t_end);
	}
#endif
}

// ------------------------------------------------------------ recompute
// Listed tokens of a large-T forward (their activations left the f16 range
// of the matrix-core path; usually none), each recomputed whole in TIE's
// exact arithmetic by one workgroup: thread per (row of F): for each slot,
// the gate and up row sums over the blocks in order (each block's dot as
// in decode_gu_kernel), SwiGLU into LDS; then thread per row of d: y_j =
// serial block sum, out = [res +] sum_j fma(g_j, y_j, .) in slot order --
// the same operations as decode_gu_kernel / decode_down_kernel, one kernel
// instead of two, so the (usually empty) launch costs once.
template <int TG, int TU, int TD>
__device__ __forceinline__ void recompute_tokens(const DecodeArgs &a, float *dl, int first, int stride)
{
	const int nbd = a.d / QK, nbf = a.F / QK, k = a.k;
	float *xs = dl;                          // [nbd][XSEG]
	float *hs = dl + (size_t)nbd * XSEG;     // [nbf][XSEG]: h of one slot
	float *acc = hs + (size_t)nbf * XSEG;    // [d]: the combine of the slots so far
	const int n = list_count(a);
	for (int li = first; li < n; li += stride) {
		const int t = list_token(a, li);
		copy_in<4>(reinterpret_cast<const float4 *>(a.x + (size_t)t * a.d), a.d / 4, [&](int q, float4 v) {
			const int f = 4 * q;
			*reinterpret_cast<float4 *>(xs + (f / QK) * XSEG + (f % QK)) = v;
		});
		for (int r = threadIdx.x; r < a.d; r += blockDim.x)
			acc[r] = 0.0f;
		__syncthreads();
		// one slot at a time: h_j in LDS, then y_j and acc = fma(g_j, y_j,
		// acc) per row (slot order, as the combine)
		for (int j = 0; j < k; j++) {
			const int e = a.topk_idx[(size_t)t * k + j];
			if (e < 0)
				continue;
			for (int r = threadIdx.x; r < a.F; r += blockDim.x) {
				float g = 0.0f, up = 0.0f;
				for (int b = 0; b < nbd; b++) {
					const uint8_t *bg = panel_slot(a.w[0], a.expert_bytes[0], e, r, b, nbd, panel_bytes(TG));
					g = g + row_block_dot<TG>(bg, q6k_d_of(bg, r), (dfloat *)(xs + b * XSEG));
				}
				for (int b = 0; b < nbd; b++) {
					const uint8_t *bu = panel_slot(a.w[1], a.expert_bytes[1], e, r, b, nbd, panel_bytes(TU));
					up = up + row_block_dot<TU>(bu, q6k_d_of(bu, r), (dfloat *)(xs + b * XSEG));
				}
				hs[(r / QK) * XSEG + r % QK] = tie_swiglu(g, up, a.silu);
			}
			__syncthreads();
			const float gw = a.topk_w[(size_t)t * k + j];
			for (int r = threadIdx.x; r < a.d; r += blockDim.x) {
				float y = 0.0f;
				for (int b = 0; b < nbf; b++) {
					const uint8_t *bd = panel_slot(a.w[2], a.expert_bytes[2], e, r, b, nbf, panel_bytes(TD));
					y = y + row_block_dot<TD>(bd, q6k_d_of(bd, r), (dfloat *)(hs + (size_t)b * XSEG));
				}
				acc[r] = __builtin_fmaf(gw, y, acc[r]);
			}
			__syncthreads();
		}
		for (int r = threadIdx.x; r < a.d; r += blockDim.x) {
			const size_t o = (size_t)t * a.d + r;
			a.out[o] = a.res ? a.res[o] + acc[r] : acc[r];
		}
		__syncthreads();
	}
}

// LDS of recompute_tokens: x, one slot's h, the combine accumulators
static size_t recompute_lds(const Layer &L)
{
	return sizeof(float) * (((size_t)(L.d / QK) + (size_t)(L.F / QK)) * XSEG + (size_t)L.d);
}

template <int TG, int TU, int TD>
__global__ __launch_bounds__(DEC_MAX_THREADS) void recompute_kernel(DecodeArgs a)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	recompute_tokens<TG, TU, TD>(a, dl, blockIdx.x, gridDim.x);
}

// The matrix-core path's last launch: the combine of every token not listed
// for recomputation (combine8_cols: out[t][c] = [res +] sum_j fma(g_j,
// y_j[c], .) in slot order, y fp32 or f16 scaled by 2^-y_shift), and, in
// workgroups of their own, the exact recomputation of the listed ones
// (usually none) -- one launch instead of two.  Workgroups [0, ncomb):
// token b / cpt, 2048 columns each (8 per thread); [ncomb, ncomb + nfix):
// recomputation.
struct CombineFixArgs {
	int ncomb, cpt, nfix;
	float ysc; // 2^y_shift
	const float *topk_w;
	const int32_t *topk_idx;
	const uint16_t *y16; // f16 y (TIE_MFMA_Y16), or
	const float *y32;    // fp32 y
	const int32_t *skip;
};
constexpr int CF_THREADS = 256;
template <int TG, int TU, int TD>
__global__ __launch_bounds__(CF_THREADS) void combine_fix_kernel(DecodeArgs a, CombineFixArgs c)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	const int b = blockIdx.x;
	if (b >= c.ncomb) {
		recompute_tokens<TG, TU, TD>(a, dl, b - c.ncomb, c.nfix);
		return;
	}
	const int t = b / c.cpt;
	// 8 columns per thread, 16-byte loads of y (d is a multiple of 256)
	const int c8 = (b - t * c.cpt) * CF_THREADS + threadIdx.x;
	if (c.skip[t] || c8 * 8 >= a.d)
		return;
	if (c.y16)
		combine8_cols<true>(t, c8, a.d, a.k, c.topk_w, c.topk_idx, c.y16, c.ysc, a.res, a.out);
	else
		combine8_cols<false>(t, c8, a.d, a.k, c.topk_w, c.topk_idx, c.y32, 1.0f, a.res, a.out);
}

// ---------------------------------------------------------------- launchers

static int round64(int n)
{
	return (n + 63) & ~63;
}

// rows per workgroup: the largest power of two <= rmax (and <= 64) whose
// tasks x rows fit one workgroup
static int pick_rows(int ntask, int rmax, int max_threads = DEC_MAX_THREADS)
{
	int R = rmax;
	while (R > 1 && ntask * R > max_threads)
		R >>= 1;
	return R;
}

// rows per gate/up and down workgroup of the one-token kernels
static int gu_rows(int nbd)
{
	return pick_rows(2 * nbd, 16);
}
static int dn_rows(int k, int nbf)
{
	return pick_rows(k * nbf, 8);
}

bool decode_supported(const Layer &L, int k)
{
	const bool q = (L.gate.type == TIE_GGML_Q4_K || L.gate.type == TIE_GGML_Q6_K) &&
		       (L.up.type == TIE_GGML_Q4_K || L.up.type == TIE_GGML_Q6_K) &&
		       (L.down.type == TIE_GGML_Q4_K || L.down.type == TIE_GGML_Q6_K);
	const int nbd = L.d / QK, nbf = L.F / QK;
	// LDS: x of one token, or the k h vectors, plus the partial dots
	const size_t lds_gu = sizeof(float) * ((size_t)nbd * XSEG + 2 * nbd * 64);
	const size_t lds_dn = sizeof(float) * ((size_t)k * nbf * XSEG + (size_t)k * nbf * 8);
	return q && k <= MAX_K && 2 * nbd <= DEC_MAX_THREADS && k * nbf <= DEC_MAX_THREADS && lds_gu <= DEC_MAX_LDS &&
	       lds_dn <= DEC_MAX_LDS;
}

template <typename K, typename... A>
static hipError_t dec_launch(K kern, dim3 grid, dim3 block, size_t lds, hipStream_t s, A... args)
{
	hipError_t err = ensure_lds_limit((const void *)kern, lds);
	if (err != hipSuccess)
		return err;
	tie_launch(kern, grid, block, lds, s, args...);
	return hipGetLastError();
}

bool recompute_supported(const Layer &L, int k)
{
	return decode_supported(L, k) && recompute_lds(L) <= DEC_MAX_LDS;
}

// The listed tokens (*count of them, their selection in topk_idx / topk_w)
// recomputed exactly into out (recompute_kernel); T bounds the list.
hipError_t launch_recompute(const Layer &L, const float *x, int k, const float *silu, const int32_t *topk_idx,
			    const float *topk_w, float *out, const float *res, const int32_t *list,
			    const int32_t *count, int T, hipStream_t s)
{
	DecodeArgs a;
	memset(&a, 0, sizeof a);
	a.w[0] = L.gate.data;
	a.w[1] = L.up.data;
	a.w[2] = L.down.data;
	a.expert_bytes[0] = L.gate.expert_bytes;
	a.expert_bytes[1] = L.up.expert_bytes;
	a.expert_bytes[2] = L.down.expert_bytes;
	a.d = L.d;
	a.F = L.F;
	a.E = L.E;
	a.k = k;
	a.x = x;
	a.topk_idx = const_cast<int32_t *>(topk_idx);
	a.topk_w = const_cast<float *>(topk_w);
	a.out = out;
	a.res = res;
	a.silu = silu;
	a.list = list;
	a.count = count;
	const size_t lds = recompute_lds(L);
	const dim3 grid(T < 128 ? (T > 0 ? T : 1) : 128);
	const int tg = L.gate.type, tu = L.up.type, td = L.down.type;
	hipError_t err;
	prof_begin("recompute", s);
#define REC(A, B)                                                                                                    \
	(td == TIE_GGML_Q4_K ? dec_launch(recompute_kernel<A, B, TIE_GGML_Q4_K>, grid, dim3(DEC_MAX_THREADS), lds, s, a) \
			     : dec_launch(recompute_kernel<A, B, TIE_GGML_Q6_K>, grid, dim3(DEC_MAX_THREADS), lds, s, a))
	if (tg == TIE_GGML_Q4_K && tu == TIE_GGML_Q4_K)
		err = REC(TIE_GGML_Q4_K, TIE_GGML_Q4_K);
	else if (tg == TIE_GGML_Q4_K)
		err = REC(TIE_GGML_Q4_K, TIE_GGML_Q6_K);
	else if (tu == TIE_GGML_Q4_K)
		err = REC(TIE_GGML_Q6_K, TIE_GGML_Q4_K);
	else
		err = REC(TIE_GGML_Q6_K, TIE_GGML_Q6_K);
#undef REC
	prof_end(s);
	return err;
}

// One launch for the combine and the recomputation when the latter's LDS
// leaves the combine workgroups their occupancy (measured: 30B shapes gain
// 6 us at T = 128 and 1.4 us at T = 2048; 235B T = 1024, 39 KiB, loses 2 us)
bool combine_fix_preferred(const Layer &L)
{
	return recompute_lds(L) <= 24 * 1024;
}

// The combine of the matrix-core path's f16 y (tokens listed in skip left
// alone) and the exact recomputation of the listed tokens, in one launch.
hipError_t launch_combine_fix(const Layer &L, const float *x, int k, const float *silu, const int32_t *topk_idx,
			      const float *topk_w, const void *y, bool y16, int y_shift, float *out, const float *res,
			      const int32_t *skip, const int32_t *list, const int32_t *count, int T, hipStream_t s)
{
	if (T == 0)
		return hipSuccess;
	DecodeArgs a;
	memset(&a, 0, sizeof a);
	a.w[0] = L.gate.data;
	a.w[1] = L.up.data;
	a.w[2] = L.down.data;
	a.expert_bytes[0] = L.gate.expert_bytes;
	a.expert_bytes[1] = L.up.expert_bytes;
	a.expert_bytes[2] = L.down.expert_bytes;
	a.d = L.d;
	a.F = L.F;
	a.E = L.E;
	a.k = k;
	a.x = x;
	a.topk_idx = const_cast<int32_t *>(topk_idx);
	a.topk_w = const_cast<float *>(topk_w);
	a.out = out;
	a.res = res;
	a.silu = silu;
	a.list = list;
	a.count = count;
	CombineFixArgs c;
	c.cpt = (L.d / 8 + CF_THREADS - 1) / CF_THREADS;
	c.ysc = ldexpf(1.0f, y_shift);
	c.ncomb = T * c.cpt;
	c.nfix = T < 64 ? T : 64;
	c.topk_w = topk_w;
	c.topk_idx = topk_idx;
	c.y16 = y16 ? reinterpret_cast<const uint16_t *>(y) : nullptr;
	c.y32 = y16 ? nullptr : reinterpret_cast<const float *>(y);
	c.skip = skip;
	const size_t lds = recompute_lds(L);
	const dim3 grid(c.ncomb + c.nfix);
	const int tg = L.gate.type, tu = L.up.type, td = L.down.type;
	hipError_t err;
	prof_begin("combine", s);
#define CF(A, B)                                                                                                     \
	(td == TIE_GGML_Q4_K ? dec_launch(combine_fix_kernel<A, B, TIE_GGML_Q4_K>, grid, dim3(CF_THREADS), lds, s, a, c) \
			     : dec_launch(combine_fix_kernel<A, B, TIE_GGML_Q6_K>, grid, dim3(CF_THREADS), lds, s, a, c))
	if (tg == TIE_GGML_Q4_K && tu == TIE_GGML_Q4_K)
		err = CF(TIE_GGML_Q4_K, TIE_GGML_Q4_K);
	else if (tg == TIE_GGML_Q4_K)
		err = CF(TIE_GGML_Q4_K, TIE_GGML_Q6_K);
	else if (tu == TIE_GGML_Q4_K)
		err = CF(TIE_GGML_Q6_K, TIE_GGML_Q4_K);
	else
		err = CF(TIE_GGML_Q6_K, TIE_GGML_Q6_K);
#undef CF
	prof_end(s);
	return err;
}

// The block for listed tokens (list == null: token 0 of a one-token call,
// routed here from its logits when inline_route) in TIE's exact arithmetic.
// h: [max_entries][k][F] scratch.  max_entries bounds the grid's list
// dimension (entries beyond it are looped over).
hipError_t launch_decode(const Layer &L, const float *x, int k, const float *silu, const float *logits,
			 int32_t *topk_idx, float *topk_w, float *h, float *out, const float *res, const int32_t *list,
			 const int32_t *count, int max_entries, bool inline_route, bool fixup, hipStream_t s)
{
	DecodeArgs a;
	memset(&a, 0, sizeof a);
	a.w[0] = L.gate.data;
	a.w[1] = L.up.data;
	a.w[2] = L.down.data;
	a.expert_bytes[0] = L.gate.expert_bytes;
	a.expert_bytes[1] = L.up.expert_bytes;
	a.expert_bytes[2] = L.down.expert_bytes;
	a.d = L.d;
	a.F = L.F;
	a.E = L.E;
	a.k = k;
	a.x = x;
	a.logits = logits;
	a.topk_idx = topk_idx;
	a.topk_w = topk_w;
	a.h = h;
	a.out = out;
	a.res = res;
	a.silu = silu;
	a.list = list;
	a.count = count;
	a.routing = L.routing;
	a.pbias = L.pbias;
	// a token list runs with one workgroup row per slot and loops over its
	// entries (usually none: the launch must stay cheap)
	const int nz = list ? 1 : (max_entries < 1 ? 1 : max_entries > 64 ? 64 : max_entries);
	const int nbd = L.d / QK, nbf = L.F / QK;
	hipError_t err;
	prof_begin(fixup ? "fixup_gate_up" : "decode_gate_up", s);
	{
		DecodeArgs g = a;
		g.R = gu_rows(nbd);
		const int threads = round64(2 * nbd * g.R);
		const size_t lds = sizeof(float) * ((size_t)nbd * XSEG + 2 * nbd * g.R);
		const dim3 grid(L.F / g.R, k, nz);
		const int tg = L.gate.type, tu = L.up.type;
#define DEC_GU(A, B)                                                                                                 \
	(inline_route ? dec_launch(decode_gu_kernel<A, B, true>, grid, dim3(threads), lds, s, g)                        \
		      : dec_launch(decode_gu_kernel<A, B, false>, grid, dim3(threads), lds, s, g))
		if (tg == TIE_GGML_Q4_K && tu == TIE_GGML_Q4_K)
			err = DEC_GU(TIE_GGML_Q4_K, TIE_GGML_Q4_K);
		else if (tg == TIE_GGML_Q4_K)
			err = DEC_GU(TIE_GGML_Q4_K, TIE_GGML_Q6_K);
		else if (tu == TIE_GGML_Q4_K)
			err = DEC_GU(TIE_GGML_Q6_K, TIE_GGML_Q4_K);
		else
			err = DEC_GU(TIE_GGML_Q6_K, TIE_GGML_Q6_K);
#undef DEC_GU
	}
	prof_end(s);
	if (err != hipSuccess)
		return err;
	prof_begin(fixup ? "fixup_down" : "decode_down", s);
	{
		DecodeArgs g = a;
		g.R = dn_rows(k, nbf);
		const int threads = round64(k * nbf * g.R);
		const size_t lds = sizeof(float) * ((size_t)k * nbf * XSEG + (size_t)k * nbf * g.R);
		const dim3 grid(L.d / g.R, 1, nz);
		err = L.down.type == TIE_GGML_Q4_K
			      ? dec_launch(decode_down_kernel<TIE_GGML_Q4_K>, grid, dim3(threads), lds, s, g)
			      : dec_launch(decode_down_kernel<TIE_GGML_Q6_K>, grid, dim3(threads), lds, s, g);
	}
	prof_end(s);
	return err;
}

// ------------------------------------------------------------ one launch: launcher
// Shape of the one-launch decode with LP lanes per (row, block) dot.
// gate/up: rg rows, 2 nb tasks per row; down: rd rows, k nb tasks per row
// (powers of two); router: rpr rows.
static void one_shape(const Layer &L, int k, int LP, int &rpr, int &rg, int &rd, int &threads, size_t &lds)
{
	const int nbd = L.d / QK, nbf = L.F / QK;
	rg = pick_rows(LP * 2 * nbd, 16);
	rd = pick_rows(LP * k * nbf, 8);
	threads = round64(std::max(std::max(LP * 2 * nbd * rg, LP * k * nbf * rd), L.E));
	rpr = L.d <= 2048 ? 2 : 1;
	const size_t lds_r = sizeof(float) * (size_t)(1 + rpr) * lane_major_floats(L.d);
	const size_t lds_g = sizeof(float) * ((size_t)nbd * XSEG + 2 * nbd * rg);
	const size_t lds_d = sizeof(float) * ((size_t)k * nbf * XSEG + (size_t)k * nbf * rd);
	lds = std::max(lds_r, std::max(lds_g, lds_d));
}

// compute units of the current device (cached per device)
static int device_cus()
{
	static int cus[64];
	int dev = 0;
	if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
		return 0;
	if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
		cus[dev] = 0;
	return cus[dev];
}

// Two lanes per dot when every workgroup of that form is resident at once
// (by waves per SIMD and by LDS per CU): the dots' latency halves, while a
// grid that does not fit would start its down workgroups only as gate/up
// ones retire, so their weights would no longer stream during gate/up.
// debug override of the choice (-1: by the shape, 0: one lane per dot, 1:
// lane pairs where the shape allows them)
static int g_one_force_form = -1;

static bool one_pairs(const Layer &L, int k)
{
	if (g_one_force_form == 0)
		return false;
	int rpr, rg, rd, threads;
	size_t lds;
	one_shape(L, k, 2, rpr, rg, rd, threads, lds);
	if (threads > DEC_MAX_THREADS || lds > DEC_MAX_LDS)
		return false;
	if (g_one_force_form == 1)
		return true;
	const long wgs = (L.E + rpr - 1) / rpr + (long)(L.F / rg) * k + L.d / rd;
	const long waves_wg = threads / 64;
	const long per_cu = std::min((long)(4 * ONE_PAIR_WAVES) / waves_wg, (long)((160 * 1024) / std::max(lds, (size_t)1)));
	return wgs <= per_cu * device_cus();
}

#ifndef TIE_ONE_MAX_D
#define TIE_ONE_MAX_D 1048576
#endif
bool decode_one_supported(const Layer &L, int k)
{
	if (!decode_supported(L, k) || L.E > INLINE_E || L.d > TIE_ONE_MAX_D)
		return false;
	int rpr, rg, rd, threads;
	size_t lds;
	one_shape(L, k, 1, rpr, rg, rd, threads, lds);
	return threads <= DEC_MAX_THREADS && lds <= DEC_MAX_LDS && 8 * rpr <= threads;
}

int decode_one_gate_up_groups(const Layer &L, int k)
{
	int rpr, rg, rd, threads;
	size_t lds;
	one_shape(L, k, one_pairs(L, k) ? 2 : 1, rpr, rg, rd, threads, lds);
	return (L.F / rg) * k;
}

hipError_t launch_decode_one(const Layer &L, const float *x, int k, const float *silu, int32_t *topk_idx,
			     float *topk_w, float *out, const float *res, unsigned long long *lg, size_t lg_copy,
			     unsigned long long *hw, size_t hw_copy, uint32_t seq, uint32_t wseq, int spin, int32_t *status,
			     hipStream_t s)
{
	OneArgs o;
	memset(&o, 0, sizeof o);
	DecodeArgs &a = o.a;
	a.w[0] = L.gate.data;
	a.w[1] = L.up.data;
	a.w[2] = L.down.data;
	a.expert_bytes[0] = L.gate.expert_bytes;
	a.expert_bytes[1] = L.up.expert_bytes;
	a.expert_bytes[2] = L.down.expert_bytes;
	a.d = L.d;
	a.F = L.F;
	a.E = L.E;
	a.k = k;
	a.x = x;
	a.topk_idx = topk_idx;
	a.topk_w = topk_w;
	a.out = out;
	a.res = res;
	a.silu = silu;
	a.routing = L.routing;
	a.pbias = L.pbias;
	int threads;
	size_t lds;
	const bool pair = one_pairs(L, k);
	one_shape(L, k, pair ? 2 : 1, o.rpr, o.rg, o.rd, threads, lds);
	o.router = L.router;
	o.bias = L.bias;
	o.lg = lg;
	o.hw = hw;
	o.lg_copy = lg_copy;
	o.hw_copy = hw_copy;
	o.seq = seq;
	o.wseq = wseq;
	o.spin = spin;
	o.status = status;
	o.nr = (L.E + o.rpr - 1) / o.rpr;
	o.ng = (L.F / o.rg) * k;
	const int nd = L.d / o.rd;
	const dim3 grid(o.nr + o.ng + nd);
	const int tg = L.gate.type, tu = L.up.type, td = L.down.type;
	hipError_t err;
	prof_begin("decode_one", s);
#define ONE_P(A, B, C)                                                                                               \
	(pair ? dec_launch(decode_one_kernel<A, B, C, true>, grid, dim3(threads), lds, s, o)                             \
	      : dec_launch(decode_one_kernel<A, B, C, false>, grid, dim3(threads), lds, s, o))
#define ONE(A, B) (td == TIE_GGML_Q4_K ? ONE_P(A, B, TIE_GGML_Q4_K) : ONE_P(A, B, TIE_GGML_Q6_K))
	if (tg == TIE_GGML_Q4_K && tu == TIE_GGML_Q4_K)
		err = ONE(TIE_GGML_Q4_K, TIE_GGML_Q4_K);
	else if (tg == TIE_GGML_Q4_K)
		err = ONE(TIE_GGML_Q4_K, TIE_GGML_Q6_K);
	else if (tu == TIE_GGML_Q4_K)
		err = ONE(TIE_GGML_Q6_K, TIE_GGML_Q4_K);
	else
		err = ONE(TIE_GGML_Q6_K, TIE_GGML_Q6_K);
#undef ONE
#undef ONE_P
	prof_end(s);
	return err;
}

// ------------------------------------------------------------ dense, few tokens
// dispatch_mat_mat (math_dispatch.c:304-359) for T <= DENSE_ROWS_T tokens
// through TIE's row kernel (mat_vec_row_f32_{q4k,q6k}_f32_avx2) as the
// decode kernels do it: a lane per (row, block) of R rows of the matrix,
// the block in registers (every load up front) and its dot taken with each
// token's x from LDS; then the serial sums over the blocks, out[t][row].
constexpr int DENSE_ROWS_T = 4;
template <int TW>
__device__ __forceinline__ void dense_rows_tile(const uint8_t *__restrict__ W, const float *__restrict__ x, int T, int in,
						int rows, int R, float *__restrict__ out, int r0, float *dl)
{
	const int nb = in / QK;
	float *xs = dl;                        // [T][nb][XSEG]
	float *part = dl + (size_t)T * nb * XSEG; // [T][nb][R]
	// the thread's first block is requested before the inputs are staged,
	// so the two memory waits overlap (unconditionally: a conditional load
	// would be waited for at once)
	RowBlock<TW> rb;
	{
		const int u = (int)threadIdx.x < nb * R ? (int)threadIdx.x : nb * R - 1;
		const int r = u & (R - 1), b = u / R;
		const uint8_t *blk = panel_slot(W, 0, 0, r0 + r, b, nb, panel_bytes(TW));
		rb.load(blk, q6k_d_of(blk, r0 + r));
	}
	copy_in<4>(reinterpret_cast<const float4 *>(x), T * in / 4, [&](int q, float4 v) {
		const int f = 4 * q, t = f / in, r = f - t * in;
		*reinterpret_cast<float4 *>(xs + ((size_t)t * nb + r / QK) * XSEG + (r % QK)) = v;
	});
	__syncthreads();
	for (int u = threadIdx.x; u < nb * R; u += blockDim.x) {
		const int r = u & (R - 1), b = u / R;
		if (u != (int)threadIdx.x) {
			const uint8_t *blk = panel_slot(W, 0, 0, r0 + r, b, nb, panel_bytes(TW));
			rb.load(blk, q6k_d_of(blk, r0 + r));
		}
		for (int t = 0; t < T; t++)
			part[((size_t)t * nb + b) * R + r] = rb.dot((dfloat *)(xs + ((size_t)t * nb + b) * XSEG));
	}
	__syncthreads();
	for (int u = threadIdx.x; u < T * R; u += blockDim.x) {
		const int t = u / R, r = u - t * R;
		float acc = 0.0f;
#pragma unroll 8
		for (int b = 0; b < nb; b++)
			acc = acc + part[((size_t)t * nb + b) * R + r];
		out[(size_t)t * rows + r0 + r] = acc;
	}
}

template <int TW> __global__ __launch_bounds__(DEC_MAX_THREADS) void dense_rows_kernel(const uint8_t *__restrict__ W,
											  const float *__restrict__ x, int T,
											  int in, int rows, int R,
											  float *__restrict__ out)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	dense_rows_tile<TW>(W, x, T, in, rows, R, out, blockIdx.x * R, dl);
}

// The exact rows (TIE's row kernel, as dense_rows_kernel) of the tokens
// flagged by the matrix-core dense path (x outside the f16 range; usually
// none), over R rows per workgroup: each workgroup walks the flags 64 at a
// time and recomputes its rows of every flagged token.
template <int TW> __global__ __launch_bounds__(DEC_MAX_THREADS) void dense_fix_kernel(const uint8_t *__restrict__ W,
											 const float *__restrict__ x, int T,
											 int in, int rows, int R,
											 float *__restrict__ out,
											 const int32_t *__restrict__ flag)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	__shared__ unsigned long long sbits;
	// usually nothing is flagged: one pass over all the flags first
	int any = 0;
	for (int i = threadIdx.x; i < T / 4; i += blockDim.x) {
		const int4 f = reinterpret_cast<const int4 *>(flag)[i];
		any |= f.x | f.y | f.z | f.w;
	}
	for (int t = (T & ~3) + threadIdx.x; t < T; t += blockDim.x)
		any |= flag[t];
	if (!__syncthreads_or(any))
		return;
	for (int t0 = 0; t0 < T; t0 += 64) {
		if (threadIdx.x < 64) {
			const int t = t0 + threadIdx.x;
			const unsigned long long m = __ballot(t < T && flag[t] != 0);
			if (threadIdx.x == 0)
				sbits = m;
		}
		__syncthreads();
		unsigned long long m = sbits;
		__syncthreads();
		while (m) {
			const int t = t0 + __builtin_ctzll(m);
			m &= m - 1;
			dense_rows_tile<TW>(W, x + (size_t)t * in, 1, in, rows, R, out + (size_t)t * rows, blockIdx.x * R, dl);
			__syncthreads();
		}
	}
}

// ------------------------------------------------------------ dense, one token, many rows
// dispatch_mat_mat (math_dispatch.c:304-359) at T = 1 for tall matrices (the
// LM head): persistent waves stream units of `rpw` rows x nb blocks, one
// lane per (row, block), and load the next unit's blocks into registers
// while the current unit's are dotted (TIE's row kernel per block, as
// dense_rows_kernel).  Each row's sum over its blocks (0 + p_0 + p_1 + ...,
// math_avx2.c:762-766) is taken in block order by the row's block-0 lane.
#ifndef TIE_STREAM_WAVES
#define TIE_STREAM_WAVES 4
#endif
constexpr int STREAM_WAVES = TIE_STREAM_WAVES;
#ifndef TIE_STREAM_PX
#define TIE_STREAM_PX 1
#endif
constexpr bool STREAM_PX = TIE_STREAM_PX;

// 0 + p_0 + p_1 + ... + p_{N-1} over lanes i .. i + N - 1 (on lane i, N <= 16
// lanes inside one DPP row), with the values brought over by row shifts.
template <int N> __device__ __forceinline__ float row_serial_sum(float p)
{
	float acc = 0.0f + p;
	if constexpr (N > 1) acc = acc + dppf<0x101>(p);
	if constexpr (N > 2) acc = acc + dppf<0x102>(p);
	if constexpr (N > 3) acc = acc + dppf<0x103>(p);
	if constexpr (N > 4) {
		acc = acc + dppf<0x104>(p);
		acc = acc + dppf<0x105>(p);
		acc = acc + dppf<0x106>(p);
		acc = acc + dppf<0x107>(p);
	}
	if constexpr (N > 8) {
		acc = acc + dppf<0x108>(p);
		acc = acc + dppf<0x109>(p);
		acc = acc + dppf<0x10a>(p);
		acc = acc + dppf<0x10b>(p);
		acc = acc + dppf<0x10c>(p);
		acc = acc + dppf<0x10d>(p);
		acc = acc + dppf<0x10e>(p);
		acc = acc + dppf<0x10f>(p);
	}
	return acc;
}

template <int TW>
__device__ __forceinline__ void stream_unit(RowBlock<TW> &cur, RowBlock<TW> &nxt, const uint8_t *__restrict__ W,
					    dfloat *xb, int u, int nu, int units, int rpw, int rl, int b, int nb, int rows,
					    float *__restrict__ out)
{
	// (unconditional: past the end every wave reads the last unit again,
	// from the cache; a conditional load would make the compiler move the
	// whole block between registers)
	const size_t pb = panel_bytes(TW);
	int row = (nu < units ? nu : units - 1) * rpw + rl;
	row = row < rows ? row : rows - 1;
	const uint8_t *blk = panel_slot(W, 0, 0, row, b, nb, pb);
	nxt.load(blk, q6k_d_of(blk, row));
	const float p = cur.template dot<STREAM_PX>(xb);
	float acc;
	switch (nb) {
	case 4: acc = row_serial_sum<4>(p); break;
	case 8: acc = row_serial_sum<8>(p); break;
	case 16: acc = row_serial_sum<16>(p); break;
	default:
		acc = 0.0f;
		for (int j = 0; j < nb; j++)
			acc = acc + __shfl(p, rl * nb + j);
	}
	row = u * rpw + rl;
	if (b == 0 && rl < rpw && row < rows)
		out[row] = acc;
}

template <int TW>
__global__ __launch_bounds__(64 * STREAM_WAVES) void dense_stream_kernel(const uint8_t *__restrict__ W,
									  const float *__restrict__ x, int in, int rows,
									  int rpw, int units, float *__restrict__ out)
{
	extern __shared__ __attribute__((aligned(16))) float dl[];
	const int nb = in / QK;
	copy_in<4>(reinterpret_cast<const float4 *>(x), in / 4, [&](int q, float4 v) {
		const int f = 4 * q;
		*reinterpret_cast<float4 *>(dl + (f / QK) * XSEG + (f % QK)) = v;
	});
	__syncthreads();
	const int lane = threadIdx.x & 63;
	const int rl = lane / nb, b = lane - rl * nb;
	dfloat *xb = (dfloat *)(dl + b * XSEG);
	const int nw = gridDim.x * STREAM_WAVES;
	// consecutive units to the waves of a workgroup, so that the waves with
	// one unit more than the others sit on different SIMDs of few CUs
	int u = blockIdx.x * STREAM_WAVES + (threadIdx.x >> 6);
	if (u >= units)
		return;
	const size_t pb = panel_bytes(TW);
	RowBlock<TW> A, B;
	{
		int row = u * rpw + rl;
		row = row < rows ? row : rows - 1;
		const uint8_t *blk = panel_slot(W, 0, 0, row, b, nb, pb);
		A.load(blk, q6k_d_of(blk, row));
	}
	for (;;) {
		stream_unit<TW>(A, B, W, xb, u, u + nw, units, rpw, rl, b, nb, rows, out);
		u += nw;
		if (u >= units)
			break;
		stream_unit<TW>(B, A, W, xb, u, u + nw, units, rpw, rl, b, nb, rows, out);
		u += nw;
		if (u >= units)
			break;
	}
}

// units of the streamed kernel at least (below it, dense_rows_kernel)
constexpr int STREAM_MIN_UNITS = 4096;

bool dense_stream_supported(const ExpertTensor &W, int T)
{
	const int nb = W.in / QK;
	return T == 1 && (W.type == TIE_GGML_Q4_K || W.type == TIE_GGML_Q6_K) && nb <= 64 &&
	       (long)W.rows * nb / 64 >= STREAM_MIN_UNITS;
}

hipError_t launch_dense_stream(const ExpertTensor &W, const float *x, float *out, hipStream_t s)
{
	const int nb = W.in / QK;
	const int rpw = 64 / nb;
	const int units = (W.rows + rpw - 1) / rpw;
	const size_t lds = sizeof(float) * (size_t)nb * XSEG;
	const void *fn = W.type == TIE_GGML_Q4_K ? (const void *)dense_stream_kernel<TIE_GGML_Q4_K>
						 : (const void *)dense_stream_kernel<TIE_GGML_Q6_K>;
	static int ncu = 0;
	if (!ncu) {
		int dev = 0;
		if (hipGetDevice(&dev) != hipSuccess ||
		    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
			ncu = 256;
	}
	int occ = 0;
	if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, 64 * STREAM_WAVES, lds) != hipSuccess || occ <= 0)
		occ = 1;
	int grid = ncu * occ;
	const int need = (units + STREAM_WAVES - 1) / STREAM_WAVES;
	grid = grid < need ? grid : need;
	return W.type == TIE_GGML_Q4_K
		       ? dec_launch(dense_stream_kernel<TIE_GGML_Q4_K>, dim3(grid), dim3(64 * STREAM_WAVES), lds, s, W.data,
				    x, W.in, W.rows, rpw, units, out)
		       : dec_launch(dense_stream_kernel<TIE_GGML_Q6_K>, dim3(grid), dim3(64 * STREAM_WAVES), lds, s, W.data,
				    x, W.in, W.rows, rpw, units, out);
}

bool dense_rows_supported(const ExpertTensor &W, int T)
{
	const int nb = W.in / QK;
	const size_t lds = sizeof(float) * ((size_t)DENSE_ROWS_T * nb * XSEG + (size_t)DENSE_ROWS_T * nb * 64);
	return T <= DENSE_ROWS_T && (W.type == TIE_GGML_Q4_K || W.type == TIE_GGML_Q6_K) && nb <= DEC_MAX_THREADS &&
	       lds <= DEC_MAX_LDS;
}

hipError_t launch_dense_fix(const ExpertTensor &W, const float *x, int T, float *out, const int32_t *flag, hipStream_t s)
{
	const int nb = W.in / QK;
	int R = 64;
	while (R > 1 && (nb * R > DEC_MAX_THREADS || W.rows / R < 512))
		R >>= 1;
	const size_t lds = sizeof(float) * ((size_t)nb * XSEG + (size_t)nb * R);
	const dim3 grid(W.rows / R);
	const dim3 block((nb * R + 63) & ~63);
	return W.type == TIE_GGML_Q4_K
		       ? dec_launch(dense_fix_kernel<TIE_GGML_Q4_K>, grid, block, lds, s, W.data, x, T, W.in, W.rows, R, out, flag)
		       : dec_launch(dense_fix_kernel<TIE_GGML_Q6_K>, grid, block, lds, s, W.data, x, T, W.in, W.rows, R, out, flag);
}

hipError_t launch_dense_rows(const ExpertTensor &W, const float *x, int T, float *out, hipStream_t s)
{
	const int nb = W.in / QK;
	// rows per workgroup: at most 64 and a workgroup's worth of lanes, and
	// few enough that the grid has ~512 workgroups (small matrices)
	int R = 64;
	while (R > 1 && (nb * R > DEC_MAX_THREADS || W.rows / R < 512))
		R >>= 1;
	const size_t lds = sizeof(float) * ((size_t)T * nb * XSEG + (size_t)T * nb * R);
	const dim3 grid(W.rows / R);
	const dim3 block((nb * R + 63) & ~63);
	return W.type == TIE_GGML_Q4_K
		       ? dec_launch(dense_rows_kernel<TIE_GGML_Q4_K>, grid, block, lds, s, W.data, x, T, W.in, W.rows, R, out)
		       : dec_launch(dense_rows_kernel<TIE_GGML_Q6_K>, grid, block, lds, s, W.data, x, T, W.in, W.rows, R, out);
}

} // namespace tie

// Debug: force the one-launch decode's form (0 a lane per dot, 1 lane pairs
// where the shape allows them; -1 chosen by the shape)
extern "C" void tie_hip_debug_decode_form(int form)
{
	tie::g_one_force_form = form;
}

#ifdef TIE_ONE_TRACE
extern "C" int tie_hip_debug_one_trace(unsigned long long *host, int reset)
{
	const size_t n = sizeof(unsigned long long) * tie::ONE_TRACE_WG * 8;
	if (hipMemcpyFromSymbol(host, HIP_SYMBOL(tie::g_one_trace), n) != hipSuccess)
		return -1;
	if (reset) {
		static unsigned long long z[tie::ONE_TRACE_WG * 8];
		if (hipMemcpyToSymbol(HIP_SYMBOL(tie::g_one_trace), z, n) != hipSuccess)
			return -1;
	}
	return 0;
}
#endif
