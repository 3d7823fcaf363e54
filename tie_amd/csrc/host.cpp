// host.cpp -- host-side pieces of the library that need no GPU: the SiLU
// table builder, the host build of the device expf, and error reporting.
#include <immintrin.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

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
