// tie_expf.h -- binary32 exp() that reproduces glibc's expf bit for bit.
//
// TIE's routing softmax calls libm expf (engine.c:880).  To make the gate
// weights bit-identical on the GPU, this header restates the published
// algorithm glibc uses for expf (Szabolcs Nagy's table-driven method from
// ARM optimized-routines, glibc sysdeps/ieee754/flt-32/e_expf.c): with
// N = 32, k = round(x * N/ln2), r = x * N/ln2 - k (one fused multiply-add,
// as glibc's FMA build computes it), 2^(k/N) from a 32-entry table of
// 2^(i/N), and a degree-3 polynomial in r, all in binary64, rounded once to
// binary32.  The host build of this same function is compared with the
// host's libm expf over every binary32 input in tests/test_host_abi.py.
//
// Compiles as host and device code (HIP); no libm call is involved.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define TIE_HD __host__ __device__ __forceinline__
#else
#define TIE_HD static inline
#endif

// T[i] = bits(2^(i/32) rounded to binary64) - (i << 52) / 32
#define TIE_EXP2_TABLE                                                                                 \
	{                                                                                              \
		0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,      \
		0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,  \
		0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,  \
		0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,  \
		0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,  \
		0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,  \
		0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,  \
		0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,  \
	}

TIE_HD double tie_as_double(uint64_t u)
{
	return __builtin_bit_cast(double, u);
}

TIE_HD uint64_t tie_as_u64(double d)
{
	return __builtin_bit_cast(uint64_t, d);
}

// tab: the 32 entries of TIE_EXP2_TABLE (device code passes a copy in LDS:
// a table lookup with a per-lane index is then an LDS read, not a load
// from global memory)
TIE_HD float tie_expf_tab(float x, const uint64_t *tab)
{
	const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
	const double shift = 0x1.8p+52;
	const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
	const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
	const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;

	const uint32_t ux = __builtin_bit_cast(uint32_t, x);
	const uint32_t abstop = (ux >> 20) & 0x7ff;
	if (abstop >= 0x42b) { // |x| >= 88, inf or nan
		if (ux == 0xff800000u)
			return 0.0f;
		if (abstop >= 0x7f8)
			return x + x;
		if (x > 0x1.62e42ep6f)
			return __builtin_inff();
		if (x < -0x1.9fe368p6f)
			return 0.0f;
	}
	const double xd = (double)x;
	const double z = inv_ln2_n * xd;
	double kd = z + shift;
	const uint64_t ki = tie_as_u64(kd);
	kd -= shift;
	const double r = __builtin_fma(inv_ln2_n, xd, -kd);
	uint64_t t = tab[ki % 32];
	t += ki << 47;
	const double s = tie_as_double(t);
	const double zz = __builtin_fma(c0, r, c1);
	const double r2 = r * r;
	double y = __builtin_fma(c2, r, 1.0);
	y = __builtin_fma(zz, r2, y);
	y = y * s;
	return (float)y;
}

TIE_HD float tie_expf(float x)
{
	const uint64_t tab[32] = TIE_EXP2_TABLE;
	return tie_expf_tab(x, tab);
}
