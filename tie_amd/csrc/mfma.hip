// mfma.hip -- grouped expert GEMMs on the bf16 matrix cores (large T).
//
// Reference: TIE runs every (token, expert) pair as three GEMVs
// (process_expert_task, engine.c:916-964) with no reuse of an expert's
// weights across tokens.  For large T the pairs are grouped by expert
// (dispatch.hip) and each expert's weights are dequantised once and
// multiplied against all of its tokens with v_mfma_f32_32x32x16_bf16:
//
//   gate/up:  G = X_e Wg_e^T, U = X_e Wu_e^T, h = silu_tab(G) * U  (fused)
//   down:     Y = h_e Wd_e^T, scattered to the pairs' rows of y
//
// Tiles: a workgroup (8 waves) owns up to MT = 256 pair rows of one expert
// -- a whole expert at the usual prefill load of ~T*k/E rows, so each weight
// is dequantised once per call -- and 128 weight rows (gate/up: 64 gate
// rows and the same 64 up rows, so TIE's table SwiGLU
// (swiglu_activation_f32_f32_avx2) is applied to the accumulators in
// registers; down: two 64-row panels).  K advances 64 at a time through a
// double-buffered LDS pipeline: the global loads of step k+1 are issued
// into registers before the MFMAs of step k and written to the other buffer
// after them (the B tile dequantised from the panel layout on the way), one
// barrier per step.  Waves form a 4 (M) x 2 (N) grid of 64 x 64 tiles; the
// M index runs fastest across SIMDs, so a half-full tile still keeps every
// SIMD's matrix core busy.
//
// Numerics: fp32 accumulation of bf16 products.  Q4_K/Q6_K weights are
// dequantised in fp32 exactly as TIE does (fma(q, d*sc, -dmin*m); d*sc*q)
// then rounded to bf16; activations are rounded to bf16.  With BF16 expert
// weights (already exact in bf16) the activations are split into a bf16
// high part and a bf16 remainder (two MFMAs per product), which keeps the
// products to ~16 mantissa bits; that path is HBM-bound, so the extra MFMA
// work is hidden.
#include "common.h"

namespace tie {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int MT = MFMA_MT;   // pair rows per workgroup (256)
constexpr int NT = 128;       // weight rows per workgroup
constexpr int KS = 64;        // K per stage
constexpr int LDK = KS + 8;   // LDS row stride (bf16) -- padding against bank conflicts
constexpr int MF_THREADS = 512;

__device__ __forceinline__ uint16_t bf16_bits(float f)
{
	return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// two floats -> two round-to-nearest-even bf16 in one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16(float a, float b)
{
	const f32x2 v = {a, b};
	return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

struct MfmaArgs {
	const uint8_t *w[2];     // gate/up: gate, up tensors; down: down tensor (both)
	size_t expert_bytes[2];
	int wtype;               // TIE_GGML_Q4_K / Q6_K / BF16
	int rows, in;            // per expert: weight rows, K
	const uint16_t *a16;     // A as bf16 rows (gate/up: x_bf16 [T][d] by token; down: h_bf16 [P][F] by position)
	const float *a32;        // A as fp32 rows (split mode)
	int k;                   // experts per token (token = pair / k)
	const int32_t *offsets, *pairs, *tile_e, *tile_m0, *ntiles;
	const float *silu;
	uint16_t *h16;           // gate/up out (bf16, by position)
	float *h32;              // gate/up out (fp32, by position; split mode)
	float *y;                // down out [pair][d]
};

// ------------------------------------------------------------------ staging
// Thread roles per K-step:
//   A: row tid/2 (0..255), half tid%2 -- 32 K values
//   B: panel m = tid/256, panel row i = (tid/4)%64, quarter q = tid%4 -- 16 K values
template <int TYPE, bool SPLIT> struct Pref {
	u32x4 a[SPLIT ? 8 : 4];
	u32x4 b0;       // Q4_K: scales chunk; Q6_K: ql; BF16: K 16q..16q+7
	u32x4 b1;       // Q6_K: qh; BF16: K 16q+8..16q+15
	u32x2 q4;       // Q4_K: 8 quant bytes
	uint32_t s6;    // Q6_K: the 4 scale bytes holding this thread's scale
	uint32_t d6;    // Q6_K: fp16 d
};

// B row in LDS of (panel m, panel row i).  Gate/up interleave the two
// matrices every 32 rows so that a wave's two 32-column MFMA tiles hold
// the gate and the up values of the same F columns.
__device__ __forceinline__ int b_row(bool down, int m, int i)
{
	return down ? m * 64 + i : (i >> 5) * 64 + m * 32 + (i & 31);
}

template <int TYPE, bool SPLIT>
__device__ __forceinline__ void load_step(const uint8_t *bsrc0, const uint8_t *bsrc1, const char *arow, int kk,
					  Pref<TYPE, SPLIT> &p)
{
	const int h = threadIdx.x & 1;
	// A (rows past the tile's end read row 0 -- always valid -- and are
	// zeroed when stored)
	if (!SPLIT) {
		const u32x4 *src = reinterpret_cast<const u32x4 *>(arow + ((size_t)kk * KS + 32 * h) * 2);
#pragma unroll
		for (int c = 0; c < 4; c++)
			p.a[c] = src[c];
	} else {
		const u32x4 *src = reinterpret_cast<const u32x4 *>(arow + ((size_t)kk * KS + 32 * h) * 4);
#pragma unroll
		for (int c = 0; c < 8; c++)
			p.a[c] = src[c];
	}
	// B
	const int m = threadIdx.x >> 8, i = (threadIdx.x >> 2) & 63, q = threadIdx.x & 3;
	const uint8_t *bsrc = m ? bsrc1 : bsrc0;
	if constexpr (TYPE == TIE_GGML_BF16) {
		const u32x4 *src = reinterpret_cast<const u32x4 *>(bsrc + ((size_t)kk * KS + 16 * q) * 2);
		p.b0 = src[0];
		p.b1 = src[1];
	} else {
		const uint8_t *panel = bsrc + (size_t)(kk / 4) * panel_bytes(TYPE);
		const uint8_t *lane_blk = panel + i * 16;
		if constexpr (TYPE == TIE_GGML_Q4_K) {
			// group g = kk%4 is quant bytes 32g..32g+31 = chunks 1+2g, 2+2g;
			// quarter q takes bytes 8q..8q+7 of the group
			const int g = kk & 3;
			p.b0 = *reinterpret_cast<const u32x4 *>(lane_blk);
			p.q4 = *reinterpret_cast<const u32x2 *>(lane_blk + (1 + 2 * g + (q >> 1)) * 1024 + 8 * (q & 1));
		} else {
			// half n = (kk/2)%2, quant row r = 2*(kk%2) + q/2, positions 16*(q%2)..+15
			const int n = (kk >> 1) & 1, r = 2 * (kk & 1) + (q >> 1), hl = q & 1;
			p.b0 = *reinterpret_cast<const u32x4 *>(lane_blk + (4 * n + 2 * (r & 1) + hl) * 1024);
			p.b1 = *reinterpret_cast<const u32x4 *>(lane_blk + (8 + 2 * n + hl) * 1024);
			const int sj = 8 * n + hl + 2 * r; // scale index
			p.s6 = *reinterpret_cast<const uint32_t *>(lane_blk + 12 * 1024 + 4 * (sj >> 2));
			p.d6 = reinterpret_cast<const uint16_t *>(panel + Q6K_CHUNKS * 1024)[i];
		}
	}
}

template <int TYPE, bool DOWN, bool SPLIT>
__device__ __forceinline__ void store_step(const Pref<TYPE, SPLIT> &p, bool alive, int kk, uint16_t *__restrict__ As,
					   uint16_t *__restrict__ Alo, uint16_t *__restrict__ Bs)
{
	const int tid = threadIdx.x;
	const int h = tid & 1;
	// A
	{
		uint16_t *dst = As + (tid >> 1) * LDK + 32 * h;
		if (!alive) {
#pragma unroll
			for (int c = 0; c < 4; c++) {
				reinterpret_cast<u32x4 *>(dst)[c] = u32x4{0, 0, 0, 0};
				if (SPLIT)
					reinterpret_cast<u32x4 *>(Alo + (tid >> 1) * LDK + 32 * h)[c] = u32x4{0, 0, 0, 0};
			}
		} else if (!SPLIT) {
#pragma unroll
			for (int c = 0; c < 4; c++)
				reinterpret_cast<u32x4 *>(dst)[c] = p.a[c];
		} else {
			uint16_t *dlo = Alo + (tid >> 1) * LDK + 32 * h;
#pragma unroll
			for (int c = 0; c < 8; c++) {
				const float v0 = __uint_as_float(p.a[c].x), v1 = __uint_as_float(p.a[c].y);
				const float v2 = __uint_as_float(p.a[c].z), v3 = __uint_as_float(p.a[c].w);
				const float hi0 = (float)(__bf16)v0, hi1 = (float)(__bf16)v1;
				const float hi2 = (float)(__bf16)v2, hi3 = (float)(__bf16)v3;
				reinterpret_cast<u32x2 *>(dst)[c] = u32x2{pack_bf16(hi0, hi1), pack_bf16(hi2, hi3)};
				reinterpret_cast<u32x2 *>(dlo)[c] = u32x2{pack_bf16(v0 - hi0, v1 - hi1), pack_bf16(v2 - hi2, v3 - hi3)};
			}
		}
	}
	// B
	const int m = tid >> 8, i = (tid >> 2) & 63, q = tid & 3;
	uint16_t *brow = Bs + b_row(DOWN, m, i) * LDK;
	if constexpr (TYPE == TIE_GGML_BF16) {
		reinterpret_cast<u32x4 *>(brow + 16 * q)[0] = p.b0;
		reinterpret_cast<u32x4 *>(brow + 16 * q)[1] = p.b1;
	} else if constexpr (TYPE == TIE_GGML_Q4_K) {
		// sub-blocks 2g (low nibbles, K 0..31) and 2g+1 (high nibbles, K 32..63)
		const int g = kk & 3;
		const u32x4 c0 = p.b0;
		const float d = half_bits_to_float(c0.x & 0xffffu), dmin = half_bits_to_float(c0.x >> 16);
		auto sb = [&](int j) {
			const int wi = j >> 2;
			const uint32_t wd = wi == 0 ? c0.y : (wi == 1 ? c0.z : c0.w);
			return (wd >> (8 * (j & 3))) & 0xffu;
		};
		auto scale_min = [&](int j, uint32_t &sc, uint32_t &mn) {
			if (j < 4) {
				sc = sb(j) & 63u;
				mn = sb(j + 4) & 63u;
			} else {
				sc = (sb(j + 4) & 15u) | ((sb(j - 4) >> 6) << 4);
				mn = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
			}
		};
		uint32_t sc0, m0, sc1, m1;
		scale_min(2 * g, sc0, m0);
		scale_min(2 * g + 1, sc1, m1);
		const float D0 = d * (float)sc0, M0 = -(dmin * (float)m0);
		const float D1 = d * (float)sc1, M1 = -(dmin * (float)m1);
		uint32_t lo[2], hi[2];
		lo[0] = p.q4.x & 0x0f0f0f0fu;
		lo[1] = p.q4.y & 0x0f0f0f0fu;
		hi[0] = (p.q4.x >> 4) & 0x0f0f0f0fu;
		hi[1] = (p.q4.y >> 4) & 0x0f0f0f0fu;
		// keep the masks byte-parallel so each weight is one v_cvt_f32_ubyteN
		asm volatile("" : "+v"(lo[0]), "+v"(lo[1]), "+v"(hi[0]), "+v"(hi[1]));
		uint32_t pl[4], ph[4];
#pragma unroll
		for (int j = 0; j < 4; j++) {
			const uint32_t wl = lo[j >> 1], wh = hi[j >> 1];
			const int s0 = 16 * (j & 1);
			pl[j] = pack_bf16(__builtin_fmaf((float)((wl >> s0) & 0xffu), D0, M0),
					  __builtin_fmaf((float)((wl >> (s0 + 8)) & 0xffu), D0, M0));
			ph[j] = pack_bf16(__builtin_fmaf((float)((wh >> s0) & 0xffu), D1, M1),
					  __builtin_fmaf((float)((wh >> (s0 + 8)) & 0xffu), D1, M1));
		}
		*reinterpret_cast<u32x4 *>(brow + 8 * q) = u32x4{pl[0], pl[1], pl[2], pl[3]};
		*reinterpret_cast<u32x4 *>(brow + 32 + 8 * q) = u32x4{ph[0], ph[1], ph[2], ph[3]};
	} else {
		// Q6_K: q = (ql nibble | qh bits << 4); w = (d*sc) * (q - 32), exact in fp32
		const int r = 2 * (kk & 1) + (q >> 1), hl = q & 1;
		const int n = (kk >> 1) & 1;
		const int sj = 8 * n + hl + 2 * r;
		const float W = half_bits_to_float(p.d6) * (float)(int8_t)((p.s6 >> (8 * (sj & 3))) & 0xffu);
		const float N = -32.0f * W;
		const int nsh = 4 * (r >> 1), hsh = 2 * r;
		uint32_t qv[4];
		const uint32_t qlw[4] = {p.b0.x, p.b0.y, p.b0.z, p.b0.w};
		const uint32_t qhw[4] = {p.b1.x, p.b1.y, p.b1.z, p.b1.w};
#pragma unroll
		for (int j = 0; j < 4; j++)
			qv[j] = ((qlw[j] >> nsh) & 0x0f0f0f0fu) | (((qhw[j] >> hsh) & 0x03030303u) << 4);
		asm volatile("" : "+v"(qv[0]), "+v"(qv[1]), "+v"(qv[2]), "+v"(qv[3]));
		uint32_t pk[8];
#pragma unroll
		for (int j = 0; j < 8; j++) {
			const uint32_t wd = qv[j >> 1];
			const int s0 = 16 * (j & 1);
			pk[j] = pack_bf16(__builtin_fmaf((float)((wd >> s0) & 0xffu), W, N),
					  __builtin_fmaf((float)((wd >> (s0 + 8)) & 0xffu), W, N));
		}
		*reinterpret_cast<u32x4 *>(brow + 32 * (r & 1) + 16 * hl) = u32x4{pk[0], pk[1], pk[2], pk[3]};
		*reinterpret_cast<u32x4 *>(brow + 32 * (r & 1) + 16 * hl + 8) = u32x4{pk[4], pk[5], pk[6], pk[7]};
	}
}

__device__ __forceinline__ bf16x8 lds_frag(const uint16_t *base, int row, int k)
{
	return *reinterpret_cast<const bf16x8 *>(base + row * LDK + k);
}

// ------------------------------------------------------------------ kernel
template <int TYPE, bool DOWN, bool SPLIT>
__global__ __launch_bounds__(MF_THREADS) void mfma_experts_kernel(MfmaArgs a)
{
	// split activations need a second A tile: single-buffered then (the BF16
	// path is HBM-bound, the extra barrier costs little)
	constexpr int NBUF = SPLIT ? 1 : 2;
	__shared__ __attribute__((aligned(16))) uint16_t As[NBUF][MT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Bs[NBUF][NT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Alo[1][SPLIT ? MT * LDK : 8];

	const int tile = blockIdx.y;
	if (tile >= *a.ntiles)
		return;
	const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
	const int pbase = a.offsets[e] + m0;
	const int nrows = min(MT, a.offsets[e + 1] - pbase);
	const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
	const int wm = w >> 1, wn = w & 1; // M (64-row slab) and N (64-col slab) of this wave
	const int lr = lane & 31, lk = 8 * (lane >> 5);
	const bool wave_live = 64 * wm < nrows;

	// this thread's A row and B source
	const int ar = threadIdx.x >> 1;
	const bool alive = ar < nrows;
	const size_t arow_idx = alive ? (DOWN ? (size_t)(pbase + ar) : (size_t)(a.pairs[pbase + ar] / a.k)) : 0;
	const char *arow = SPLIT ? (const char *)(a.a32 + arow_idx * a.in) : (const char *)(a.a16 + arow_idx * a.in);
	const uint8_t *bsrc[2];
	{
		const int bi = (threadIdx.x >> 2) & 63;
		const int nb = a.in / QK;
#pragma unroll
		for (int mm = 0; mm < 2; mm++) {
			const int mat = DOWN ? 0 : mm;
			const int rt = DOWN ? 2 * blockIdx.x + mm : blockIdx.x;
			const uint8_t *base = (mat ? a.w[1] : a.w[0]) + (size_t)e * (mat ? a.expert_bytes[1] : a.expert_bytes[0]);
			if (TYPE == TIE_GGML_BF16)
				bsrc[mm] = base + ((size_t)(rt * 64 + bi) * a.in) * 2;
			else
				bsrc[mm] = base + (size_t)rt * nb * panel_bytes(TYPE);
		}
	}

	f32x16 acc[4];
#pragma unroll
	for (int t = 0; t < 4; t++)
#pragma unroll
		for (int j = 0; j < 16; j++)
			acc[t][j] = 0.0f;

	auto compute = [&](int cur) {
		if (!wave_live)
			return;
		const uint16_t *A = As[cur], *B = Bs[cur];
		const uint16_t *AL = Alo[0];
#pragma unroll
		for (int s = 0; s < KS / 16; s++) {
			const bf16x8 a0 = lds_frag(A, 64 * wm + lr, 16 * s + lk);
			const bf16x8 a1 = lds_frag(A, 64 * wm + 32 + lr, 16 * s + lk);
			const bf16x8 b0 = lds_frag(B, 64 * wn + lr, 16 * s + lk);
			const bf16x8 b1 = lds_frag(B, 64 * wn + 32 + lr, 16 * s + lk);
			acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0], 0, 0, 0);
			acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[1], 0, 0, 0);
			acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[2], 0, 0, 0);
			acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[3], 0, 0, 0);
			if (SPLIT) {
				const bf16x8 l0 = lds_frag(AL, 64 * wm + lr, 16 * s + lk);
				const bf16x8 l1 = lds_frag(AL, 64 * wm + 32 + lr, 16 * s + lk);
				acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l0, b0, acc[0], 0, 0, 0);
				acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l0, b1, acc[1], 0, 0, 0);
				acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l1, b0, acc[2], 0, 0, 0);
				acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l1, b1, acc[3], 0, 0, 0);
			}
		}
	};

	const int nk = a.in / KS;
	Pref<TYPE, SPLIT> pf;
	load_step<TYPE, SPLIT>(bsrc[0], bsrc[1], arow, 0, pf);
	store_step<TYPE, DOWN, SPLIT>(pf, alive, 0, As[0], Alo[0], Bs[0]);
	__syncthreads();
	for (int kk = 0; kk < nk; kk++) {
		const int cur = NBUF == 2 ? (kk & 1) : 0;
		const int nxt = NBUF == 2 ? (cur ^ 1) : 0;
		if (kk + 1 < nk)
			load_step<TYPE, SPLIT>(bsrc[0], bsrc[1], arow, kk + 1, pf);
		compute(cur);
		if (NBUF == 1)
			__syncthreads();
		if (kk + 1 < nk)
			store_step<TYPE, DOWN, SPLIT>(pf, alive, kk + 1, As[nxt], Alo[0], Bs[nxt]);
		__syncthreads();
	}
	if (!wave_live)
		return;

	// D layout of v_mfma_f32_32x32x16: lane l, register j holds
	// row 8*(j/4) + 4*(l/32) + j%4, column l%32.
#pragma unroll
	for (int i = 0; i < 2; i++) {
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int mrow = 64 * wm + 32 * i + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
			if (mrow >= nrows)
				continue;
			const int p = pbase + mrow;
			if (!DOWN) {
				// acc[2i]: gate, acc[2i+1]: up, of F column blockIdx.x*64 + 32*wn + lr
				const int col = blockIdx.x * 64 + 32 * wn + lr;
				const float hv = tie_swiglu(acc[2 * i][j], acc[2 * i + 1][j], a.silu);
				if (SPLIT)
					a.h32[(size_t)p * a.rows + col] = hv;
				else
					a.h16[(size_t)p * a.rows + col] = bf16_bits(hv);
			} else {
				const int pair = a.pairs[p];
				float *yr = a.y + (size_t)pair * a.rows + blockIdx.x * 128 + 64 * wn + lr;
				yr[0] = acc[2 * i][j];
				yr[32] = acc[2 * i + 1][j];
			}
		}
	}
}

// x (fp32) -> bf16 rows for the gate/up A operand
__global__ void to_bf16_kernel(const float *__restrict__ x, uint16_t *__restrict__ y, size_t n4)
{
	for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
		const float4 v = reinterpret_cast<const float4 *>(x)[i];
		reinterpret_cast<uint2 *>(y)[i] = make_uint2(pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
	}
}

template <bool DOWN, bool SPLIT>
static hipError_t launch_one(const MfmaArgs &a, int type, dim3 grid, hipStream_t s)
{
	if (type == TIE_GGML_Q4_K)
		hipLaunchKernelGGL((mfma_experts_kernel<TIE_GGML_Q4_K, DOWN, SPLIT>), grid, dim3(MF_THREADS), 0, s, a);
	else if (type == TIE_GGML_Q6_K)
		hipLaunchKernelGGL((mfma_experts_kernel<TIE_GGML_Q6_K, DOWN, SPLIT>), grid, dim3(MF_THREADS), 0, s, a);
	else
		hipLaunchKernelGGL((mfma_experts_kernel<TIE_GGML_BF16, DOWN, SPLIT>), grid, dim3(MF_THREADS), 0, s, a);
	return hipGetLastError();
}

int mfma_max_tiles(int npairs, int E)
{
	return (npairs + MT - 1) / MT + E;
}

hipError_t launch_mfma_experts(const Layer &L, const float *x, int T, int k, const float *silu, Workspace &ws,
			       hipStream_t s)
{
	const int npairs = T * k;
	if (npairs == 0)
		return hipSuccess;
	// gate and up must share a type for the fused SwiGLU tile
	if (L.gate.type != L.up.type)
		return hipErrorInvalidValue;
	const bool split = L.gate.type == TIE_GGML_BF16;
	const bool split_down = L.down.type == TIE_GGML_BF16;
	MfmaArgs a;
	a.k = k;
	a.offsets = ws.offsets;
	a.pairs = ws.pairs;
	a.tile_e = ws.tile_e;
	a.tile_m0 = ws.tile_m0;
	a.ntiles = ws.ntiles;
	a.silu = silu;
	a.y = ws.y;
	const int max_tiles = mfma_max_tiles(npairs, L.E);

	prof_begin("mfma_gate_up", s);
	if (!split) {
		const size_t n4 = (size_t)T * L.d / 4;
		hipLaunchKernelGGL(to_bf16_kernel, dim3((unsigned)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096)),
				   dim3(256), 0, s, x, ws.xb, n4);
	}
	a.w[0] = L.gate.data;
	a.w[1] = L.up.data;
	a.expert_bytes[0] = L.gate.expert_bytes;
	a.expert_bytes[1] = L.up.expert_bytes;
	a.wtype = L.gate.type;
	a.rows = L.F;
	a.in = L.d;
	a.a16 = ws.xb;
	a.a32 = x;
	a.h16 = ws.hb;
	a.h32 = ws.h;
	hipError_t err = split ? launch_one<false, true>(a, L.gate.type, dim3(L.F / 64, max_tiles), s)
			       : launch_one<false, false>(a, L.gate.type, dim3(L.F / 64, max_tiles), s);
	prof_end(s);
	if (err != hipSuccess)
		return err;

	prof_begin("mfma_down", s);
	a.w[0] = a.w[1] = L.down.data;
	a.expert_bytes[0] = a.expert_bytes[1] = L.down.expert_bytes;
	a.wtype = L.down.type;
	a.rows = L.d;
	a.in = L.F;
	a.a16 = ws.hb;
	a.a32 = ws.h;
	if (split != split_down) {
		// activations were written in the gate/up path's precision; convert
		const size_t n = (size_t)npairs * L.F;
		if (split) {
			hipLaunchKernelGGL(to_bf16_kernel, dim3(4096), dim3(256), 0, s, ws.h, ws.hb, n / 4);
		} else {
			prof_end(s);
			return hipErrorInvalidValue; // bf16 h cannot feed the split down path
		}
	}
	err = split_down ? launch_one<true, true>(a, L.down.type, dim3(L.d / 128, max_tiles), s)
			 : launch_one<true, false>(a, L.down.type, dim3(L.d / 128, max_tiles), s);
	prof_end(s);
	return err;
}

} // namespace tie
