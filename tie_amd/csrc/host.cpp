// host.cpp -- host-side pieces of the library that need no GPU: the SiLU
// table builder, the host build of the device expf, and error reporting.
#include <immintrin.h>
#include <math.h>

#include <cmath>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "../../include/tie_hip.h"
#include "tie_expf.h"

namespace tie {

static thread_local char g_err[512];

int set_error(int code, const char *fmt, ...)
{
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(g_err, sizeof g_err, fmt, ap);
	va_end(ap);
	return code;
}

void clear_error()
{
	g_err[0] = 0;
}

// ------------------------------------------------------------- SiLU table
// TIE builds silu_table once at start-up (engine.c:35, silu_table_init at
// engine.c:297-303, expf_fast at :204-225) and its Makefile compiles with
// -O3 -ffast-math -fno-associative-math -ffp-contract=fast -march=native.
// Under those flags GCC vectorises the loop, replaces the division by 8191
// with a multiply by the float nearest 1/8191 fused with the -10 offset,
// contracts the Schraudolph polynomial into FMAs and turns x / (1 + e) into
// x * r' with r' one Newton step, r' = (r + r) - ((1 + e) * r) * r, on the
// CPU's approximate reciprocal r of (1 + e): VRCP14PS on an AVX-512 host,
// VRCPPS otherwise.  The approximate-reciprocal bits are a property of the
// CPU, so the table is built here on the host that runs TIE, with the same
// instruction a native build of TIE would use on it.

__attribute__((target("avx2,fma"))) static void rcp8_avx(const float *den, float *r)
{
	_mm256_storeu_ps(r, _mm256_rcp_ps(_mm256_loadu_ps(den)));
}

__attribute__((target("avx512f"))) static void rcp8_avx512(const float *den, float *r)
{
	float tmp[16];
	_mm512_storeu_ps(tmp, _mm512_rcp14_ps(_mm512_castps256_ps512(_mm256_loadu_ps(den))));
	memcpy(r, tmp, 8 * sizeof(float));
}

__attribute__((target("avx2,fma"))) static void silu_table_build(float *tab, bool avx512)
{
	const float r8191 = 1.0f / 8191.0f;
	for (int i = 0; i < TIE_SILU_TABLE_SIZE; i += 8) {
		float xs[8], den[8], rr[8];
		for (int l = 0; l < 8; l++) {
			const float x0 = (float)(i + l) * 20.0f;
			xs[l] = fmaf(x0, r8191, -10.0f);
			float c = fmaf(-x0, r8191, 10.0f);
			c = c < 88.37626266479492f ? c : 88.37626266479492f;
			c = c > -88.37626266479492f ? c : -88.37626266479492f;
			const float t = fmaf(12102203.0f, c, 1065353216.0f);
			const int32_t ui = (int32_t)t;
			float u;
			memcpy(&u, &ui, 4);
			float p = u;
			p = fmaf(1.9875691500E-4f, p, 1.3981999507E-3f) * p;
			p = fmaf(p, p, fmaf(8.3334519073E-3f, p, 4.1665795894E-2f) * p);
			p = fmaf(p, p, fmaf(1.6666665459E-1f, p, 5.0000001201E-1f) * p);
			den[l] = fmaf(u, p, u) + 1.0f;
		}
		if (avx512)
			rcp8_avx512(den, rr);
		else
			rcp8_avx(den, rr);
		for (int l = 0; l < 8; l++) {
			const float t = (den[l] * rr[l]) * rr[l];
			const float inv = (rr[l] + rr[l]) - t;
			tab[i + l] = xs[l] * inv;
		}
	}
}

int silu_table_host(float *tab, int n)
{
	if (!tab || n != TIE_SILU_TABLE_SIZE)
		return set_error(TIE_HIP_EINVAL, "silu table needs %d entries", TIE_SILU_TABLE_SIZE);
	__builtin_cpu_init();
	if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma"))
		return set_error(TIE_HIP_EINVAL, "host CPU lacks AVX2/FMA (TIE requires AVX2, engine.c:17-21)");
	silu_table_build(tab, __builtin_cpu_supports("avx512f"));
	return TIE_HIP_OK;
}

// ----------------------------------------------------------- rsqrt table
// TIE's rms_norm (rms_norm_f32_f32_f32_avx2, math_avx2.c:56-96) computes
// 1.0f / sqrtf(ss / size + eps).  Under -ffast-math GCC emits RSQRTSS and
// one Newton step: y0 = rsqrtss(a), inv = fma(a * y0, y0, -3) * (y0 * -0.5)
// (ix86's software rsqrt).  The approximate y0 is a property of the CPU, so
// the library tabulates the host's RSQRTSS: its output for a and for a * 4^s
// differ only in the exponent (checked below), so it is a function of the
// exponent parity and of the mantissa, and on the CPUs seen so far of only
// its top few bits (10 on current Intel server parts).  The table holds,
// for parity p (biased exponent 126 + p) and the top `nbits` mantissa bits
// j, the bits of rsqrtss(2^(p-1) * 1.j).

__attribute__((target("sse"))) static float rsqrtss(float a)
{
	return _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(a)));
}

static uint32_t fbits(float f)
{
	uint32_t u;
	memcpy(&u, &f, 4);
	return u;
}

static float bitsf(uint32_t u)
{
	float f;
	memcpy(&f, &u, 4);
	return f;
}

int rsqrt_table_host(std::vector<uint32_t> &tab, int &nbits)
{
	constexpr uint32_t M = 1u << 23;
	std::vector<uint32_t> all(2 * M);
	for (uint32_t p = 0; p < 2; p++)
		for (uint32_t m = 0; m < M; m++)
			all[p * M + m] = fbits(rsqrtss(bitsf(((126u + p) << 23) | m)));
	// the fewest leading mantissa bits the output depends on
	int n = 0;
	for (uint32_t p = 0; p < 2; p++)
		for (uint32_t m = 1; m < M; m++)
			if (all[p * M + m] != all[p * M + m - 1]) {
				const int need = 23 - __builtin_ctz(m);
				n = need > n ? need : n;
			}
	// exponent scaling: rsqrtss(a * 4^s) = rsqrtss(a) * 2^-s over the normal
	// range, on every mantissa of a stride that visits all index values
	for (int s = -62; s <= 64; s++) {
		for (uint32_t p = 0; p < 2; p++) {
			const int eb = 126 + (int)p + 2 * s;
			if (eb < 1 || eb > 254)
				continue;
			for (uint32_t m = 0; m < M; m += 1021) {
				const uint32_t want = all[p * M + m] - (uint32_t)(s * (1 << 23));
				if (fbits(rsqrtss(bitsf(((uint32_t)eb << 23) | m))) != want)
					return set_error(TIE_HIP_EINVAL,
							 "host RSQRTSS does not scale with the exponent (exponent %d, mantissa %u)",
							 eb, m);
			}
		}
	}
	nbits = n;
	tab.assign(2u << n, 0);
	for (uint32_t p = 0; p < 2; p++)
		for (uint32_t j = 0; j < (1u << n); j++)
			tab[(p << n) + j] = all[p * M + (j << (23 - n))];
	return TIE_HIP_OK;
}

// ------------------------------------------------------ f16 range of h
// The matrix-core path stores the SwiGLU output h as f16 times 2^-shift.
// The shift centres the layer's typical |h| at about 2^2 inside f16's
// normal range [2^-14, 2^16): 14 octaves of headroom above it (a token
// beyond them is recomputed exactly), and small activations stay normal
// numbers instead of losing bits as subnormals.  Typical |h| follows from
// the gate weights' RMS over a sample of their blocks: for inputs of unit
// RMS (RMSNorm outputs) a row dot is ~ sqrt(d) RMS(w), and h = silu(g) u
// is of the order of its square.

static float f16_host(uint16_t h)
{
	const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
	const float v = e == 0 ? ldexpf((float)m, -24) : e == 31 ? INFINITY : ldexpf((float)(m | 1024u), (int)e - 25);
	return (h & 0x8000u) ? -v : v;
}

double weight_mean_square(int type, const uint8_t *b, size_t n_bytes)
{
	double ss = 0.0;
	size_t n = 0;
	if (type == TIE_GGML_Q4_K) {
		for (size_t o = 0; o + 144 <= n_bytes; o += 144) {
			const uint8_t *blk = b + o;
			uint16_t hd, hm;
			memcpy(&hd, blk, 2);
			memcpy(&hm, blk + 2, 2);
			const float dd = f16_host(hd), dmin = f16_host(hm);
			const uint8_t *sc = blk + 4, *qs = blk + 16;
			for (int j = 0; j < 8; j++) {
				int s, m;
				if (j < 4) {
					s = sc[j] & 63;
					m = sc[j + 4] & 63;
				} else {
					s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
					m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
				}
				for (int i = 0; i < 32; i++) {
					const int q = (j & 1) ? qs[32 * (j >> 1) + i] >> 4 : qs[32 * (j >> 1) + i] & 15;
					const double w = (double)dd * s * q - (double)dmin * m;
					ss += w * w;
				}
			}
			n += 256;
		}
	} else if (type == TIE_GGML_Q6_K) {
		for (size_t o = 0; o + 210 <= n_bytes; o += 210) {
			const uint8_t *blk = b + o;
			uint16_t hd;
			memcpy(&hd, blk + 208, 2);
			const double dd = f16_host(hd);
			for (int i = 0; i < 256; i++) {
				// ql nibble and qh bits of weight i (block_q6_K order)
				const int half = i >> 7, l = i & 127, r = l >> 5, li = l & 31;
				const uint8_t ql = blk[64 * half + li + 32 * (r & 1)];
				const int lo = r < 2 ? ql & 15 : ql >> 4;
				const int hi = (blk[128 + 32 * half + li] >> (2 * r)) & 3;
				const int sc = (int8_t)blk[192 + 8 * half + li / 16 + 2 * r];
				const double w = dd * sc * ((lo | (hi << 4)) - 32);
				ss += w * w;
			}
			n += 256;
		}
	} else if (type == TIE_GGML_BF16) {
		for (size_t o = 0; o + 2 <= n_bytes; o += 2) {
			uint16_t v;
			memcpy(&v, b + o, 2);
			uint32_t u = (uint32_t)v << 16;
			float f;
			memcpy(&f, &u, 4);
			ss += (double)f * f;
			n++;
		}
	}
	if (n == 0 || !(ss > 0.0) || !std::isfinite(ss))
		return 0.0;
	return ss / (double)n;
}

// The MFMA path's f16 scales of h and y (powers of two), from mean squares
// of sampled gate and down weights, for RMS-normed inputs (|x| ~ 1):
// a gate / up row sum is ~ sqrt(d) rms(w_gate), h = silu(g) u ~ d ms_gate,
// y ~ sqrt(F) h rms(w_down).  h is stored as f16(h 2^-h_shift) with the
// typical |h| near 2^2, y as f16(y 2^-y_shift) with the typical |y| near
// 2^4: 2^14 and 2^12 below f16's largest value, 2^16 and 2^18 above its
// smallest normal one.
void f16_shifts(double ms_gate, double ms_down, int d, int F, int &h_shift, int &y_shift)
{
	auto clamp = [](int v) { return v < -24 ? -24 : v > 24 ? 24 : v; };
	if (!(ms_gate > 0.0) || !std::isfinite(ms_gate)) {
		h_shift = y_shift = 0;
		return;
	}
	const double h_typ = (double)d * ms_gate;
	h_shift = clamp((int)lrint(log2(h_typ)) - 2);
	if (!(ms_down > 0.0) || !std::isfinite(ms_down)) {
		y_shift = 0;
		return;
	}
	const double y_typ = sqrt((double)F) * h_typ * sqrt(ms_down);
	y_shift = clamp((int)lrint(log2(y_typ)) - 4);
}

} // namespace tie

extern "C" const char *tie_hip_last_error(void)
{
	return tie::g_err;
}

extern "C" int tie_hip_silu_table_host(float *table, int n)
{
	return tie::silu_table_host(table, n);
}

extern "C" void tie_hip_host_expf(const float *in, float *out, size_t n)
{
	for (size_t i = 0; i < n; i++)
		out[i] = tie_expf(in[i]);
}
