/*
 * tie_oracle.c -- CPU restatement of TIE's Qwen3-MoE FFN block.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in tie_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * What it restates (reference = szemzoa/tie, read as text):
 *   - the MoE branch of transformer_layer_qwen3      model_qwen3.c:404-471
 *   - softmax / find_top_k / process_expert_task      engine.c:864-964
 *   - silu_table_init + expf_fast                     engine.c:204-225, 297-303
 *   - the AVX2 row kernels that the dispatch table    math_dispatch.c:102-107
 *     selects for (F32 x {F32,Q4_K,Q6_K,BF16} -> F32):
 *       mat_vec_row_f32_f32_f32_avx2                  math_avx2.c:228-256
 *       dot_product_f32_q4k_avx2 / row               math_avx2.c:535-604, 753-769
 *       dot_product_f32_q6k_avx2 / row               math_avx2.c:411-495, 771-787
 *       dot_product_f32_bf16_avx2 / row              math_avx2.c:148-158, 188-226
 *       hsum_f32_avx2                                 math_avx2.c:14-21
 *       swiglu_activation_f32_f32_avx2                math_avx2.c:908-950
 *   - fp16_to_fp32, get_scale_min_k4                  math_scalar.c:46-67, 91-100
 *   - block_q4_k / block_q6_k layout                  gguf.h:100-113
 *
 * Numerical contract.  The reference is built with
 *   -O3 -mfma -mavx2 -ffast-math -fno-associative-math -ffp-contract=fast
 * (Makefile:10).  Under those flags GCC fuses some multiply/add pairs and
 * turns some divisions into reciprocal multiplies.  This restatement spells
 * every one of those decisions out (fmaf() where the compiled reference
 * fuses, a separate product where it does not, an explicit reciprocal where
 * it multiplies by one) and is itself compiled with -ffp-contract=off and
 * without -ffast-math, so the compiler adds nothing.  The 8-lane AVX2
 * accumulators are written as arrays of 8 floats so the summation tree is
 * explicit; the HIP kernels follow the same trees.
 *
 * Pinning: every function here is checked against vectors produced by the
 * compiled reference itself (tests/golden/, made by oracle/ref_driver.c
 * linked against the reference sources) and against closed forms (fp64
 * dequantised GEMV, brute-force top-k, softmax identities) in tests/.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>

#include "tie_oracle.h"

/* ------------------------------------------------------------------ */
/* format helpers                                                       */
/* ------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, exact for every input (math_scalar.c:46-67). */
float orc_fp16_to_fp32(uint16_t h)
{
	uint32_t sign = (uint32_t)(h >> 15) << 31;
	uint32_t e = (h >> 10) & 0x1f;
	uint32_t m = h & 0x3ff;
	uint32_t bits;
	if (e == 0x1f) {
		bits = sign | 0x7f800000u | (m << 13);
	} else if (e != 0) {
		bits = sign | ((e + 112u) << 23) | (m << 13);
	} else if (m != 0) {
		/* subnormal half: normalise the mantissa */
		int ex = 113;
		uint32_t mm = m << 13;
		while ((mm & 0x00800000u) == 0) {
			mm <<= 1;
			ex--;
		}
		bits = sign | ((uint32_t)ex << 23) | (mm & 0x007fffffu);
	} else {
		bits = sign;
	}
	float f;
	memcpy(&f, &bits, 4);
	return f;
}

static float bf16_bits_to_f32(uint16_t b)
{
	uint32_t bits = (uint32_t)b << 16;
	float f;
	memcpy(&f, &bits, 4);
	return f;
}

static uint16_t rd16(const uint8_t *p)
{
	return (uint16_t)(p[0] | (p[1] << 8));
}

/* Q4_K sub-block j (0..7): 6-bit scale and min (math_scalar.c:91-100). */
void orc_q4k_scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *mn)
{
	if (j < 4) {
		*sc = s[j] & 63;
		*mn = s[j + 4] & 63;
	} else {
		*sc = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
		*mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
	}
}

size_t orc_row_bytes(int type, int in_dim)
{
	switch (type) {
	case ORC_F32:
		return (size_t)in_dim * 4;
	case ORC_BF16:
		return (size_t)in_dim * 2;
	case ORC_Q4_K:
		return (size_t)(in_dim / 256) * 144;
	case ORC_Q6_K:
		return (size_t)(in_dim / 256) * 210;
	default:
		return 0;
	}
}

/* ------------------------------------------------------------------ */
/* 8-lane reductions                                                    */
/* ------------------------------------------------------------------ */

/* hsum_f32_avx2 (math_avx2.c:14-21): lo+hi, then two horizontal adds. */
static float hsum8(const float v[8])
{
	float s0 = v[0] + v[4];
	float s1 = v[1] + v[5];
	float s2 = v[2] + v[6];
	float s3 = v[3] + v[7];
	float a = s0 + s1;
	float b = s2 + s3;
	return a + b;
}

/* F32 row . F32 x (math_avx2.c:228-256): one 8-lane FMA accumulator,
 * hsum, then a scalar FMA tail. */
float orc_dot_f32(const float *x, const float *w, int n)
{
	float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	int j = 0;
	for (; j <= n - 8; j += 8)
		for (int l = 0; l < 8; l++)
			acc[l] = fmaf(x[j + l], w[j + l], acc[l]);
	float s = hsum8(acc);
	for (; j < n; j++)
		s = fmaf(x[j], w[j], s);
	return s;
}

/* BF16 row . F32 x (math_avx2.c:188-226): same tree as the F32 row. */
float orc_dot_bf16(const float *x, const uint16_t *w, int n)
{
	float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	int j = 0;
	for (; j + 8 <= n; j += 8)
		for (int l = 0; l < 8; l++)
			acc[l] = fmaf(x[j + l], bf16_bits_to_f32(w[j + l]), acc[l]);
	float s = hsum8(acc);
	for (; j < n; j++)
		s = fmaf(x[j], bf16_bits_to_f32(w[j]), s);
	return s;
}

/* One Q4_K super-block (256 weights) . x[0..255]
 * (math_avx2.c:535-604).  Two 8-lane accumulators; accumulator a0 takes
 * bytes [off, off+8) of each 32-byte quant group, a1 takes [off+8, off+16),
 * off in {0,16}; each byte feeds its low nibble (sub-block 2g) and then its
 * high nibble (sub-block 2g+1).  The dequantised weight is
 * fma(q, d*sc, -(dmin*m)) -- GCC contracts the reference's mul/sub into
 * one vfmsub. */
float orc_dot_q4k_block(const float *x, const uint8_t *blk)
{
	const float d = orc_fp16_to_fp32(rd16(blk));
	const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
	const uint8_t *sc = blk + 4;
	const uint8_t *qs = blk + 16;
	float D[8], M[8];
	for (int j = 0; j < 8; j++) {
		uint8_t s, m;
		orc_q4k_scale_min(j, sc, &s, &m);
		D[j] = d * (float)s;
		M[j] = dmin * (float)m;
	}
	float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	float a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	for (int g = 0; g < 4; g++) {
		const uint8_t *q = qs + 32 * g;
		const float *xg = x + 64 * g;
		const float D1 = D[2 * g], M1 = M[2 * g];
		const float D2 = D[2 * g + 1], M2 = M[2 * g + 1];
		for (int off = 0; off < 32; off += 16) {
			for (int l = 0; l < 8; l++) {
				uint8_t b = q[off + l];
				a0[l] = fmaf(xg[off + l], fmaf((float)(b & 15), D1, -M1), a0[l]);
				a0[l] = fmaf(xg[32 + off + l], fmaf((float)(b >> 4), D2, -M2), a0[l]);
			}
			for (int l = 0; l < 8; l++) {
				uint8_t b = q[off + 8 + l];
				a1[l] = fmaf(xg[off + 8 + l], fmaf((float)(b & 15), D1, -M1), a1[l]);
				a1[l] = fmaf(xg[32 + off + 8 + l], fmaf((float)(b >> 4), D2, -M2), a1[l]);
			}
		}
	}
	float v[8];
	for (int l = 0; l < 8; l++)
		v[l] = a0[l] + a1[l];
	return hsum8(v);
}

/* One Q6_K super-block . x[0..255] (math_avx2.c:411-495).  Per 128-half n
 * and per 8-wide step l in {0,8,16,24}: four 6-bit quants per byte
 * position, weights d*sc[is + 2i] (is = l>=16), term = fma(w, q*x, acc)
 * alternating between accumulators a0, a1, a0, a1. */
float orc_dot_q6k_block(const float *x, const uint8_t *blk)
{
	const uint8_t *ql = blk;
	const uint8_t *qh = blk + 128;
	const int8_t *sc = (const int8_t *)(blk + 192);
	const float d = orc_fp16_to_fp32(rd16(blk + 208));
	float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	float a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	for (int n = 0; n < 2; n++) {
		const float *xp = x + 128 * n;
		const uint8_t *lp = ql + 64 * n;
		const uint8_t *hp = qh + 32 * n;
		const int8_t *sp = sc + 8 * n;
		for (int l = 0; l < 32; l += 8) {
			const int is = (l >= 16) ? 1 : 0;
			const float w0 = d * (float)sp[is + 0];
			const float w1 = d * (float)sp[is + 2];
			const float w2 = d * (float)sp[is + 4];
			const float w3 = d * (float)sp[is + 6];
			for (int m = 0; m < 8; m++) {
				const int L = lp[l + m], L2 = lp[l + 32 + m], H = hp[l + m];
				const int q1 = ((L & 15) | ((H & 3) << 4)) - 32;
				const int q2 = ((L2 & 15) | (((H >> 2) & 3) << 4)) - 32;
				const int q3 = ((L >> 4) | (((H >> 4) & 3) << 4)) - 32;
				const int q4 = ((L2 >> 4) | (((H >> 6) & 3) << 4)) - 32;
				a0[m] = fmaf(w0, (float)q1 * xp[l + m], a0[m]);
				a1[m] = fmaf(w1, (float)q2 * xp[l + 32 + m], a1[m]);
				a0[m] = fmaf(w2, (float)q3 * xp[l + 64 + m], a0[m]);
				a1[m] = fmaf(w3, (float)q4 * xp[l + 96 + m], a1[m]);
			}
		}
	}
	float v[8];
	for (int l = 0; l < 8; l++)
		v[l] = a0[l] + a1[l];
	return hsum8(v);
}

/* o[r] = W[r] . x for r < rows; W row-major in GGUF layout.  Quantised rows
 * sum their per-block dots serially, starting from +0.0f
 * (math_avx2.c:753-787). */
int orc_matvec(const float *x, const void *W, int type, int in_dim, int rows, float *o)
{
	const size_t rb = orc_row_bytes(type, in_dim);
	if (rb == 0)
		return -1;
	for (int r = 0; r < rows; r++) {
		const uint8_t *row = (const uint8_t *)W + (size_t)r * rb;
		float s;
		switch (type) {
		case ORC_F32:
			s = orc_dot_f32(x, (const float *)row, in_dim);
			break;
		case ORC_BF16:
			s = orc_dot_bf16(x, (const uint16_t *)row, in_dim);
			break;
		case ORC_Q4_K:
			s = 0.0f;
			for (int b = 0; b < in_dim / 256; b++)
				s = s + orc_dot_q4k_block(x + 256 * b, row + 144 * (size_t)b);
			break;
		case ORC_Q6_K:
			s = 0.0f;
			for (int b = 0; b < in_dim / 256; b++)
				s = s + orc_dot_q6k_block(x + 256 * b, row + 210 * (size_t)b);
			break;
		default:
			return -1;
		}
		o[r] = s;
	}
	return 0;
}

/* ------------------------------------------------------------------ */
/* SiLU table and SwiGLU                                                */
/* ------------------------------------------------------------------ */

/* silu_table_init + expf_fast (engine.c:204-225, 297-303) as GCC compiles
 * them under the reference's flags: the loop is vectorised 8-wide, the
 * division by 8191 becomes a multiply by the float nearest 1/8191 fused
 * with the -10 offset, the Schraudolph polynomial is contracted into FMAs,
 * and x / (1 + e) becomes x * (one Newton step on RCPPS(1 + e)).  RCPPS is
 * an approximate instruction whose bits differ between CPU vendors, so the
 * table is a property of the host CPU: it is rebuilt on whatever host runs
 * the block, exactly as TIE rebuilds it at start-up. */
/* The reciprocal step of the table build.  TIE's Makefile compiles with
 * -march=native, so which approximate-reciprocal instruction GCC picks
 * depends on the build host: VRCP14PS when AVX-512F is available, VRCPPS
 * otherwise.  mode 1 forces RCPPS, mode 2 forces RCP14PS, 0 picks by CPUID
 * the way a native build on this host would. */
__attribute__((target("avx2,fma"))) static void rcp8_avx2(const float *den, float *r)
{
	_mm256_storeu_ps(r, _mm256_rcp_ps(_mm256_loadu_ps(den)));
}

__attribute__((target("avx512f"))) static void rcp8_avx512(const float *den, float *r)
{
	__m512 v = _mm512_castps256_ps512(_mm256_loadu_ps(den));
	float tmp[16];
	_mm512_storeu_ps(tmp, _mm512_rcp14_ps(v));
	memcpy(r, tmp, 8 * sizeof(float));
}

int orc_silu_rcp_mode(void)
{
	__builtin_cpu_init();
	return __builtin_cpu_supports("avx512f") ? 2 : 1;
}

/* silu_table_init + expf_fast (engine.c:204-225, 297-303) as GCC compiles
 * them under the reference's flags: the loop is vectorised, the division
 * by 8191 becomes a multiply by the float nearest 1/8191 fused with the -10
 * offset, the Schraudolph polynomial is contracted into FMAs, and
 * x / (1 + e) becomes x * (one Newton step on an approximate reciprocal of
 * 1 + e).  The approximate reciprocal's bits are a property of the host CPU,
 * so the table is rebuilt on whatever host runs the block, exactly as TIE
 * rebuilds it at start-up (engine.c:35). */
int orc_silu_table(float *tab, int mode)
{
	if (mode == 0)
		mode = orc_silu_rcp_mode();
	if (mode != 1 && mode != 2)
		return -1;
	if (mode == 2 && orc_silu_rcp_mode() != 2)
		return -1;
	const float r8191 = 1.0f / 8191.0f; /* 0x39000400 */
	for (int i = 0; i < ORC_SILU_N; i += 8) {
		float xs[8], den[8], rr[8];
		for (int l = 0; l < 8; l++) {
			float x0 = (float)(i + l) * 20.0f;
			xs[l] = fmaf(x0, r8191, -10.0f);
			float c = fmaf(-x0, r8191, 10.0f);
			c = c < 88.37626266479492f ? c : 88.37626266479492f;
			c = c > -88.37626266479492f ? c : -88.37626266479492f;
			float t = fmaf(12102203.0f, c, 1065353216.0f);
			int32_t ui = (int32_t)t;
			float u;
			memcpy(&u, &ui, 4);
			float p = u;
			p = fmaf(1.9875691500E-4f, p, 1.3981999507E-3f) * p;
			p = fmaf(p, p, fmaf(8.3334519073E-3f, p, 4.1665795894E-2f) * p);
			p = fmaf(p, p, fmaf(1.6666665459E-1f, p, 5.0000001201E-1f) * p);
			den[l] = fmaf(u, p, u) + 1.0f;
		}
		if (mode == 2)
			rcp8_avx512(den, rr);
		else
			rcp8_avx2(den, rr);
		for (int l = 0; l < 8; l++) {
			float t = (den[l] * rr[l]) * rr[l];
			float inv = (rr[l] + rr[l]) - t;
			tab[i + l] = xs[l] * inv;
		}
	}
	return 0;
}

/* swiglu_activation_f32_f32_avx2 (math_avx2.c:908-950): gate <- silu(gate) * up.
 * pos = ((x + 10) * 8191) * 0.05f  (the /20 is a reciprocal multiply),
 * idx = round-half-even(pos) with CVTPS2DQ's out-of-range result INT_MIN,
 * clamped to [0, 8190]; linear interpolation with one FMA.  Outside
 * [-10, 10] the end segments are extrapolated, not saturated. */
void orc_swiglu(float *gate, const float *up, int n, const float *tab)
{
	for (int i = 0; i < n; i++) {
		float x = gate[i];
		float pos = ((x + 10.0f) * 8191.0f) * 0.05f;
		int32_t idx;
		if (pos >= -2147483648.0f && pos < 2147483648.0f)
			idx = (int32_t)nearbyintf(pos);
		else
			idx = INT32_MIN; /* CVTPS2DQ "integer indefinite" (NaN / overflow) */
		if (idx < 0)
			idx = 0;
		if (idx > ORC_SILU_N - 2)
			idx = ORC_SILU_N - 2;
		float frac = pos - (float)idx;
		float y1 = tab[idx], y2 = tab[idx + 1];
		float s = fmaf(frac, y2 - y1, y1);
		gate[i] = s * up[i];
	}
}

/* ------------------------------------------------------------------ */
/* routing                                                              */
/* ------------------------------------------------------------------ */

/* find_top_k (engine.c:891-914): keeps the k largest logits in descending
 * order; an incoming logit enters only if strictly greater than the current
 * k-th, and moves up only past strictly smaller ones, so among equal logits
 * the lower expert index ranks first.  NaN and -inf never enter; unfilled
 * slots stay {-1, -inf}. */
void orc_find_top_k(const float *logits, int E, int k, int32_t *idx, float *score)
{
	for (int s = 0; s < k; s++) {
		idx[s] = -1;
		score[s] = -INFINITY;
	}
	for (int e = 0; e < E; e++) {
		float v = logits[e];
		if (!(v > score[k - 1]))
			continue;
		int pos = k - 1;
		while (pos > 0 && v > score[pos - 1]) {
			idx[pos] = idx[pos - 1];
			score[pos] = score[pos - 1];
			pos--;
		}
		idx[pos] = e;
		score[pos] = v;
	}
}

/* softmax over the k selected logits (engine.c:864-888): max, expf (libm),
 * serial sum, then a multiply by 1/sum (the division is turned into a
 * reciprocal multiply by -ffast-math). */
void orc_softmax(float *v, int n)
{
	if (n == 0)
		return;
	float mx = v[0];
	for (int i = 1; i < n; i++)
		if (v[i] > mx)
			mx = v[i];
	float sum = 0.0f;
	for (int i = 0; i < n; i++) {
		v[i] = expf(v[i] - mx);
		sum = sum + v[i];
	}
	float inv = 1.0f / sum;
	for (int i = 0; i < n; i++)
		v[i] = v[i] * inv;
}

/* LFM2 routing (model_lfm2.c:437-467): p_e = 1 / (1 + expf(-l_e)) (libm
 * expf, IEEE division); top-k (find_top_k) over p_e + bias_e (bias
 * optional); the weights are the unbiased p of the selected experts over
 * their serial sum + 1e-6, as a multiply by the reciprocal.  Unfilled
 * slots (index -1) get weight 0 (TIE would read scores[-1]). */
void orc_sigmoid_route(const float *logits, int E, int k, const float *probs_bias, int32_t *idx, float *w)
{
	float p[1024], sel[1024];
	for (int e = 0; e < E; e++) {
		p[e] = 1.0f / (1.0f + expf(-logits[e]));
		sel[e] = probs_bias ? p[e] + probs_bias[e] : p[e];
	}
	float score[ORC_MAX_K];
	orc_find_top_k(sel, E, k, idx, score);
	float sum = 0.0f;
	for (int j = 0; j < k; j++) {
		w[j] = idx[j] >= 0 ? p[idx[j]] : 0.0f;
		sum = sum + w[j];
	}
	float inv = 1.0f / (sum + 1e-6f);
	for (int j = 0; j < k; j++)
		w[j] = w[j] * inv;
}

/* ------------------------------------------------------------------ */
/* the block                                                            */
/* ------------------------------------------------------------------ */

/* Byte offset of expert e inside a stacked [E][rows][in] expert tensor.
 * TIE computes it as e * rows * (in/256) * ggml_block_size(type)
 * (engine.c:929-942); for BF16 ggml_block_size is 2 (gguf.c:28-29), which
 * under-counts by a factor 256.  literal != 0 reproduces that. */
static size_t expert_offset(int type, int rows, int in_dim, int e, int literal)
{
	if (literal && type == ORC_BF16)
		return (size_t)e * rows * (size_t)(in_dim / 256) * 2;
	return (size_t)e * rows * orc_row_bytes(type, in_dim);
}

static int type_ok(int t)
{
	return t == ORC_Q4_K || t == ORC_Q6_K || t == ORC_BF16;
}

int orc_moe_block(const float *x, int T, int d, int F, int E, int k, const float *router_w,
		  const float *router_bias, int routing, const float *probs_bias, const void *gate_w, int gate_type, const void *up_w, int up_type,
		  const void *down_w, int down_type, int literal_bf16_stride, const float *silu_tab, float *out,
		  int32_t *topk_idx, float *topk_w, float *logits_out, int nthreads)
{
	if (T < 0 || d <= 0 || F <= 0 || E <= 0 || E > 1024 || k <= 0 || k > E || k > ORC_MAX_K)
		return -1;
	if (routing != 0 && routing != 1)
		return -1;
	if (d % 256 || F % 256)
		return -1;
	if (!type_ok(gate_type) || !type_ok(up_type) || !type_ok(down_type))
		return -1;
	if (nthreads < 1)
		nthreads = 1;

#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
	for (int t = 0; t < T; t++) {
		const float *xt = x + (size_t)t * d;
		float *logits = (float *)malloc(sizeof(float) * E);
		float *h1 = (float *)malloc(sizeof(float) * F);
		float *h2 = (float *)malloc(sizeof(float) * F);
		float *y = (float *)malloc(sizeof(float) * d);
		float *acc = out + (size_t)t * d;

		/* router logits (model_qwen3.c:431-432) */
		orc_matvec(xt, router_w, ORC_F32, d, E, logits);
		if (router_bias)
			for (int e = 0; e < E; e++)
				logits[e] = logits[e] + router_bias[e];
		if (logits_out)
			memcpy(logits_out + (size_t)t * E, logits, sizeof(float) * E);

		int32_t sel[ORC_MAX_K];
		float g[ORC_MAX_K];
		if (routing == 1) {
			orc_sigmoid_route(logits, E, k, probs_bias, sel, g);
		} else {
			orc_find_top_k(logits, E, k, sel, g);
			orc_softmax(g, k);
		}

		memset(acc, 0, sizeof(float) * d);
		for (int j = 0; j < k; j++) {
			int e = sel[j];
			if (e < 0 || e >= E) {
				/* TIE would index out of bounds here; the restatement
				 * treats an unfilled slot as contributing nothing. */
				continue;
			}
			const uint8_t *wg = (const uint8_t *)gate_w + expert_offset(gate_type, F, d, e, literal_bf16_stride);
			const uint8_t *wu = (const uint8_t *)up_w + expert_offset(up_type, F, d, e, literal_bf16_stride);
			const uint8_t *wd = (const uint8_t *)down_w + expert_offset(down_type, d, F, e, literal_bf16_stride);
			orc_matvec(xt, wg, gate_type, d, F, h1);
			orc_matvec(xt, wu, up_type, d, F, h2);
			orc_swiglu(h1, h2, F, silu_tab);
			orc_matvec(h1, wd, down_type, F, d, y);
			/* combine (model_qwen3.c:459-467): out += g_j * y_j, fused */
			for (int c = 0; c < d; c++)
				acc[c] = fmaf(g[j], y[c], acc[c]);
		}
		if (topk_idx)
			memcpy(topk_idx + (size_t)t * k, sel, sizeof(int32_t) * k);
		if (topk_w)
			memcpy(topk_w + (size_t)t * k, g, sizeof(float) * k);
		free(logits);
		free(h1);
		free(h2);
		free(y);
	}
	return 0;
}

/* rms_norm_f32_f32_f32_avx2 (math_avx2.c:56-96) as TIE's build computes it
 * (our build of the reference sources, read back): eight FMA chains over
 * x[8i + l], the hsum tree, ss / size + eps, then 1/sqrtf as GCC emits it
 * under -ffast-math: y0 = RSQRTSS(a) on this host (the instruction itself,
 * as TIE runs it) and one Newton step fma(a*y0, y0, -3) * (y0 * -0.5);
 * out = (x * w) * inv. */
__attribute__((target("avx2,fma"))) void orc_rms_norm(const float *x, const float *w, int size, float eps, float *o)
{
	float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
	int i = 0;
	for (; i <= size - 8; i += 8)
		for (int l = 0; l < 8; l++)
			acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
	float ss = hsum8(acc);
	for (; i < size; i++)
		ss = fmaf(x[i], x[i], ss);
	const float a = ss / (float)size + eps;
	const float y0 = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(a)));
	const float inv = fmaf(a * y0, y0, -3.0f) * (y0 * -0.5f);
	for (i = 0; i < size; i++)
		o[i] = (x[i] * w[i]) * inv;
}

/* The FFN half of transformer_layer_qwen3: RMSNorm of every token
 * (model_qwen3.c:392-401), the MoE block (:404-471), then the residual add
 * hidden += ffn_down_output (:491, apply_residual_f32_f32_avx2,
 * math_avx2.c:731-751).  hidden is updated in place. */
int orc_qwen3_ffn(float *hidden, int T, int d, int F, int E, int k, const float *ffn_norm, float eps,
		  const float *router_w, const void *gate_w, int gate_type, const void *up_w, int up_type,
		  const void *down_w, int down_type, const float *silu_tab, int32_t *topk_idx, float *topk_w,
		  int nthreads)
{
	if (T < 0 || d <= 0)
		return -1;
	float *normed = (float *)calloc((size_t)(T > 0 ? T : 1) * d, sizeof(float));
	float *out = (float *)calloc((size_t)(T > 0 ? T : 1) * d, sizeof(float));
	for (int t = 0; t < T; t++)
		orc_rms_norm(hidden + (size_t)t * d, ffn_norm, d, eps, normed + (size_t)t * d);
	int rc = orc_moe_block(normed, T, d, F, E, k, router_w, NULL, 0, NULL, gate_w, gate_type, up_w, up_type,
			       down_w, down_type, 0, silu_tab, out, topk_idx, topk_w, NULL, nthreads);
	if (rc == 0)
		for (size_t i = 0; i < (size_t)T * d; i++)
			hidden[i] = hidden[i] + out[i];
	free(normed);
	free(out);
	return rc;
}

/* ------------------------------------------------------------------ */
/* dequantisers (closed-form checks)                                    */
/* ------------------------------------------------------------------ */

/* dequantize_row_q4_k_f32_scalar (math_scalar.c:216-255). */
void orc_dequant_q4k(const uint8_t *blocks, int n, float *y)
{
	for (int b = 0; b < n / 256; b++) {
		const uint8_t *blk = blocks + 144 * (size_t)b;
		const float d = orc_fp16_to_fp32(rd16(blk));
		const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
		for (int g = 0; g < 4; g++) {
			uint8_t s1, m1, s2, m2;
			orc_q4k_scale_min(2 * g, blk + 4, &s1, &m1);
			orc_q4k_scale_min(2 * g + 1, blk + 4, &s2, &m2);
			for (int l = 0; l < 32; l++) {
				uint8_t q = blk[16 + 32 * g + l];
				y[256 * b + 64 * g + l] = (d * s1) * (float)(q & 15) - dmin * m1;
				y[256 * b + 64 * g + 32 + l] = (d * s2) * (float)(q >> 4) - dmin * m2;
			}
		}
	}
}

/* dequantize_row_q6_k_f32_scalar (math_scalar.c:257-288). */
void orc_dequant_q6k(const uint8_t *blocks, int n, float *y)
{
	for (int b = 0; b < n / 256; b++) {
		const uint8_t *blk = blocks + 210 * (size_t)b;
		const float d = orc_fp16_to_fp32(rd16(blk + 208));
		const int8_t *sc = (const int8_t *)(blk + 192);
		for (int h = 0; h < 2; h++) {
			const uint8_t *ql = blk + 64 * h;
			const uint8_t *qh = blk + 128 + 32 * h;
			float *yy = y + 256 * b + 128 * h;
			for (int l = 0; l < 32; l++) {
				int is = l / 16;
				int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
				int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
				int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
				int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
				yy[l] = d * sc[8 * h + is + 0] * q1;
				yy[l + 32] = d * sc[8 * h + is + 2] * q2;
				yy[l + 64] = d * sc[8 * h + is + 4] * q3;
				yy[l + 96] = d * sc[8 * h + is + 6] * q4;
			}
		}
	}
}

/* libm expf over an array: the function TIE's softmax calls
 * (engine.c:880), exposed so tests can compare other expf implementations
 * with it. */
void orc_expf_array(const float *in, float *out, size_t n)
{
	for (size_t i = 0; i < n; i++)
		out[i] = expf(in[i]);
}
