// norm.hip -- the RMSNorm in front of the MoE block (model_qwen3.c:392-401).
//
// rms_norm_f32_f32_f32_avx2 (math_avx2.c:56-96) as TIE's build computes it:
//   ss  = hsum8 of eight FMA chains, chain l over x[8i + l] (i ascending)
//   a   = ss / size + eps                       (IEEE divide and add)
//   y0  = RSQRTSS(a)                            (the host CPU's approximation)
//   inv = fma(a * y0, y0, -3) * (y0 * -0.5)     (GCC's Newton step)
//   out = (x * w) * inv
// RSQRTSS comes from a table built on the host at set-up (its output depends
// only on the exponent parity and the top `nbits` mantissa bits; the
// exponent scales exactly), so the kernel reproduces TIE's bits.
#include "common.h"
#include "route.h"

namespace tie {

// the host's RSQRTSS of a positive normal float through the table
__device__ __forceinline__ float rsqrt_host(float a, const uint32_t *tab, int nbits)
{
	const uint32_t b = __builtin_bit_cast(uint32_t, a);
	const int eb = (int)(b >> 23);
	if (eb == 0)
		return __builtin_inff(); // zero (eps = 0 and an all-zero row)
	const int p = (eb - 126) & 1;
	const int s = (eb - 126 - p) >> 1;
	const uint32_t y = tab[(p << nbits) + ((b & 0x7fffffu) >> (23 - nbits))];
	return __builtin_bit_cast(float, y - (uint32_t)(s * (1 << 23)));
}

// One wave per token.  The wave stages the row in LDS a chunk at a time
// with coalesced 16-byte loads, stored by chain: chain l's elements x[8i +
// l] are contiguous (row stride padded by 4 floats, so the 16-byte reads of
// lanes 0..7 fall in different banks); lanes 0..7 then run the eight
// sum-of-squares chains four elements per LDS read.  Then the whole wave
// scales the row.
constexpr int NORM_THREADS = 256;
constexpr int NORM_CHUNK = 2048;               // floats of a row staged per wave at a time
constexpr int NORM_LSTRIDE = NORM_CHUNK / 8 + 4; // floats per chain row in LDS
__global__ __launch_bounds__(NORM_THREADS) void rmsnorm_kernel(const float *__restrict__ x,
							     const float *__restrict__ w, float eps, int T, int d,
							     float *__restrict__ out, const uint32_t *__restrict__ tab,
							     int nbits)
{
	__shared__ __attribute__((aligned(16))) float rows[NORM_THREADS / 64][8 * NORM_LSTRIDE];
	const int wave = threadIdx.x >> 6;
	const int t = blockIdx.x * (NORM_THREADS / 64) + wave;
	if (t >= T)
		return;
	const int lane = threadIdx.x & 63;
	const float *xr = x + (size_t)t * d;
	float *buf = rows[wave];
	float acc = 0.0f;
	for (int c0 = 0; c0 < d; c0 += NORM_CHUNK) {
		const int n = d - c0 < NORM_CHUNK ? d - c0 : NORM_CHUNK; // a multiple of 256
		for (int c = 4 * lane; c < n; c += 256) {
			const float4 v = *reinterpret_cast<const float4 *>(xr + c0 + c);
			// element c + j goes to chain (c + j) % 8, position (c + j) / 8
			const int l = c & 7, i = c >> 3;
			buf[(l + 0) * NORM_LSTRIDE + i] = v.x;
			buf[(l + 1) * NORM_LSTRIDE + i] = v.y;
			buf[(l + 2) * NORM_LSTRIDE + i] = v.z;
			buf[(l + 3) * NORM_LSTRIDE + i] = v.w;
		}
		__builtin_amdgcn_wave_barrier();
		__builtin_amdgcn_s_waitcnt(0);
		__builtin_amdgcn_wave_barrier();
		if (lane < 8) {
			const float *ch = buf + lane * NORM_LSTRIDE;
#pragma unroll 4
			for (int i = 0; i < n / 8; i += 4) {
				const float4 v = *reinterpret_cast<const float4 *>(ch + i);
				acc = __builtin_fmaf(v.x, v.x, acc);
				acc = __builtin_fmaf(v.y, v.y, acc);
				acc = __builtin_fmaf(v.z, v.z, acc);
				acc = __builtin_fmaf(v.w, v.w, acc);
			}
		}
		__builtin_amdgcn_wave_barrier();
	}
	const float ss = hsum8_lanes(acc); // lane 0
	float inv = 0.0f;
	if (lane == 0) {
		const float a = __fdiv_rn(ss, (float)d) + eps;
		const float y0 = rsqrt_host(a, tab, nbits);
		inv = __builtin_fmaf(a * y0, y0, -3.0f) * (y0 * -0.5f);
	}
	inv = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, inv)));
	float *o = out + (size_t)t * d;
	for (int c = 4 * lane; c < d; c += 256) {
		const float4 xv = *reinterpret_cast<const float4 *>(xr + c);
		const float4 wv = *reinterpret_cast<const float4 *>(w + c);
		float4 r;
		r.x = (xv.x * wv.x) * inv;
		r.y = (xv.y * wv.y) * inv;
		r.z = (xv.z * wv.z) * inv;
		r.w = (xv.w * wv.w) * inv;
		*reinterpret_cast<float4 *>(o + c) = r;
	}
}

hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int T, int d, float *out, const uint32_t *tab,
			  int nbits, hipStream_t s)
{
	if (T == 0)
		return hipSuccess;
	tie_launch(rmsnorm_kernel, dim3((T + NORM_THREADS / 64 - 1) / (NORM_THREADS / 64)), dim3(NORM_THREADS),
			   0, s, x, w, eps, T, d, out, tab, nbits);
	return hipGetLastError();
}

} // namespace tie
