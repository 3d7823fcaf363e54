// mfma.hip -- grouped expert GEMMs on the bf16 matrix cores (large T).
//
// Reference: TIE runs every (token, expert) pair as three GEMVs
// (process_expert_task, engine.c:916-964) with no reuse of an expert's
// weights across tokens.  For large T the pairs are grouped by expert
// (dispatch.hip) and each expert's weights are dequantised once per tile and
// multiplied against all of its tokens with v_mfma_f32_32x32x16_bf16:
//
//   gate/up:  G = X_e Wg_e^T, U = X_e Wu_e^T, h = silu_tab(G) * U  (fused)
//   down:     Y = h_e Wd_e^T, scattered to the pairs' rows of y
//
// Tiles: a workgroup (4 waves) owns MT = 128 pair rows of one expert and
// 128 weight rows (gate: 64 gate + the same 64 up rows, so the SwiGLU of
// TIE's swiglu_activation_f32_f32_avx2 is applied to the accumulators in
// registers; down: two 64-row panels).  K advances 64 at a time: the A tile
// (bf16 activations, gathered by pair) is copied into LDS and the B tile is
// dequantised from the panel layout straight into LDS as bf16.  Wave w
// multiplies A rows 32w..32w+31 by the four 32-row B tiles.
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
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int MT = 128;       // pair rows per workgroup
constexpr int NT = 128;       // weight rows per workgroup
constexpr int KS = 64;        // K per stage
constexpr int LDK = KS + 8;   // LDS row stride (bf16) -- padding against bank conflicts
constexpr int MF_THREADS = 256;

__device__ __forceinline__ uint16_t bf16_bits(float f)
{
	return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b)
{
	return (uint32_t)bf16_bits(a) | ((uint32_t)bf16_bits(b) << 16);
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
// Each K-step moves a 128 x 64 A tile and a 128 x 64 B tile into LDS.  The
// global loads of step kk+1 are issued into registers before the MFMAs of
// step kk (Pref), and written to the other LDS buffer (with the B dequant)
// after them, so HBM latency overlaps the matrix work: one barrier per step.
//
// Thread roles: A -- row tid/2, half tid%2 (32 K values); B -- panel
// m = tid/128, panel row i = (tid/2)%64, half h = tid%2.
template <int TYPE, bool SPLIT> struct Pref {
	u32x4 a[SPLIT ? 8 : 4];
	u32x4 b[TYPE == TIE_GGML_Q4_K ? 2 : TYPE == TIE_GGML_Q6_K ? 5 : 4];
	uint32_t d6;
};

// B row in LDS of (panel m, panel row i).  Gate/up interleave the two
// matrices every 32 rows so that a wave's two 32-column MFMA tiles hold
// the gate and the up values of the same F columns.
__device__ __forceinline__ int b_row(bool down, int m, int i)
{
	return down ? m * 64 + i : (i >> 5) * 64 + m * 32 + (i & 31);
}

template <int TYPE, bool DOWN, bool SPLIT>
__device__ __forceinline__ void load_step(const MfmaArgs &a, const uint8_t *bsrc0, const uint8_t *bsrc1, const char *arow, bool alive,
					  int kk, Pref<TYPE, SPLIT> &p)
{
	const int h = threadIdx.x & 1;
	// A (rows past the tile's end read row 0 -- always valid -- and are
	// zeroed when stored)
	(void)alive;
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
	const int m = threadIdx.x >> 7, i = (threadIdx.x >> 1) & 63;
	if constexpr (TYPE == TIE_GGML_BF16) {
		const u32x4 *src = reinterpret_cast<const u32x4 *>((m ? bsrc1 : bsrc0) + ((size_t)kk * KS + 32 * h) * 2);
#pragma unroll
		for (int c = 0; c < 4; c++)
			p.b[c] = src[c];
	} else {
		const uint8_t *panel = (m ? bsrc1 : bsrc0) + (size_t)(kk / 4) * panel_bytes(TYPE);
		const u32x4 *pc = reinterpret_cast<const u32x4 *>(panel) + i;
		if constexpr (TYPE == TIE_GGML_Q4_K) {
			const int g = kk & 3;
			p.b[0] = pc[0];
			p.b[1] = pc[(1 + 2 * g + h) * 64];
		} else {
			const int n = (kk >> 1) & 1, r = 2 * (kk & 1) + h;
			p.b[0] = pc[(4 * n + 2 * (r & 1)) * 64];
			p.b[1] = pc[(4 * n + 2 * (r & 1) + 1) * 64];
			p.b[2] = pc[(8 + 2 * n) * 64];
			p.b[3] = pc[(9 + 2 * n) * 64];
			p.b[4] = pc[12 * 64];
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
				reinterpret_cast<uint4 *>(dst)[c] = make_uint4(0, 0, 0, 0);
				if (SPLIT)
					reinterpret_cast<uint4 *>(Alo + (tid >> 1) * LDK + 32 * h)[c] = make_uint4(0, 0, 0, 0);
			}
		} else if (!SPLIT) {
#pragma unroll
			for (int c = 0; c < 4; c++)
				reinterpret_cast<u32x4 *>(dst)[c] = p.a[c];
		} else {
			uint16_t *dlo = Alo + (tid >> 1) * LDK + 32 * h;
#pragma unroll
			for (int c = 0; c < 8; c++) {
				const float4 v = make_float4(__uint_as_float(p.a[c].x), __uint_as_float(p.a[c].y),
							     __uint_as_float(p.a[c].z), __uint_as_float(p.a[c].w));
				const float hi0 = (float)(__bf16)v.x, hi1 = (float)(__bf16)v.y;
				const float hi2 = (float)(__bf16)v.z, hi3 = (float)(__bf16)v.w;
				reinterpret_cast<uint2 *>(dst)[c] = make_uint2(pack_bf16(hi0, hi1), pack_bf16(hi2, hi3));
				reinterpret_cast<uint2 *>(dlo)[c] =
					make_uint2(pack_bf16(v.x - hi0, v.y - hi1), pack_bf16(v.z - hi2, v.w - hi3));
			}
		}
	}
	// B
	const int m = tid >> 7, i = (tid >> 1) & 63;
	uint16_t *brow = Bs + b_row(DOWN, m, i) * LDK;
	if constexpr (TYPE == TIE_GGML_BF16) {
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<u32x4 *>(brow + 32 * h)[c] = p.b[c];
	} else if constexpr (TYPE == TIE_GGML_Q4_K) {
		// K slice = group g (sub-blocks 2g, 2g+1); half h = bytes 16h..16h+15 of the group
		const int g = kk & 3;
		const u32x4 c0 = p.b[0], q = p.b[1];
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
		const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
		uint32_t lo[8], hi[8];
#pragma unroll
		for (int j = 0; j < 8; j++) {
			const uint32_t b0 = (qw[j >> 1] >> (16 * (j & 1))) & 0xffu;
			const uint32_t b1 = (qw[j >> 1] >> (16 * (j & 1) + 8)) & 0xffu;
			lo[j] = pack_bf16(__builtin_fmaf((float)(b0 & 15u), D0, M0), __builtin_fmaf((float)(b1 & 15u), D0, M0));
			hi[j] = pack_bf16(__builtin_fmaf((float)(b0 >> 4), D1, M1), __builtin_fmaf((float)(b1 >> 4), D1, M1));
		}
		uint16_t *d0 = brow + 16 * h; // lo nibbles: K 16h..16h+15; hi nibbles: 32+16h..
		reinterpret_cast<uint4 *>(d0)[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
		reinterpret_cast<uint4 *>(d0)[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
		reinterpret_cast<uint4 *>(d0 + 32)[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
		reinterpret_cast<uint4 *>(d0 + 32)[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
	} else {
		// Q6_K: K slice = half n of the block, quant row r = 2*(kk&1) + h
		// (elements 32r + l); w = (d * sc) * (q - 32), exact in fp32
		const int n = (kk >> 1) & 1, r = 2 * (kk & 1) + h;
		const uint32_t qlw[8] = {p.b[0].x, p.b[0].y, p.b[0].z, p.b[0].w, p.b[1].x, p.b[1].y, p.b[1].z, p.b[1].w};
		const uint32_t qhw[8] = {p.b[2].x, p.b[2].y, p.b[2].z, p.b[2].w, p.b[3].x, p.b[3].y, p.b[3].z, p.b[3].w};
		const float d = half_bits_to_float(p.d6);
		auto scale = [&](int j) {
			const int wi = j >> 2;
			const uint32_t wd = wi == 0 ? p.b[4].x : (wi == 1 ? p.b[4].y : (wi == 2 ? p.b[4].z : p.b[4].w));
			return (float)(int8_t)((wd >> (8 * (j & 3))) & 0xffu);
		};
		const float W0 = d * scale(8 * n + 2 * r), W1 = d * scale(8 * n + 1 + 2 * r);
		const float N0 = -32.0f * W0, N1 = -32.0f * W1;
		const int nsh = 4 * (r >> 1), hsh = 2 * r;
		uint32_t pk[16];
#pragma unroll
		for (int j = 0; j < 16; j++) {
			float wv[2];
#pragma unroll
			for (int t = 0; t < 2; t++) {
				const int l = 2 * j + t;
				const uint32_t L = (qlw[l >> 2] >> (8 * (l & 3))) & 0xffu;
				const uint32_t H = (qhw[l >> 2] >> (8 * (l & 3))) & 0xffu;
				const uint32_t qv = ((L >> nsh) & 15u) | (((H >> hsh) & 3u) << 4);
				wv[t] = l < 16 ? __builtin_fmaf((float)qv, W0, N0) : __builtin_fmaf((float)qv, W1, N1);
			}
			pk[j] = pack_bf16(wv[0], wv[1]);
		}
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<uint4 *>(brow + 32 * h)[c] = make_uint4(pk[4 * c], pk[4 * c + 1], pk[4 * c + 2],
										 pk[4 * c + 3]);
	}
}

__device__ __forceinline__ bf16x8 lds_frag(const uint16_t *base, int row, int k)
{
	return *reinterpret_cast<const bf16x8 *>(base + row * LDK + k);
}

// ------------------------------------------------------------------ kernel
// Workgroup tile 128 pairs x 128 weight rows; 2 x 2 waves of 64 x 64, each
// a 2 x 2 grid of 32 x 32 MFMA tiles.
template <int TYPE, bool DOWN, bool SPLIT>
__global__ __launch_bounds__(MF_THREADS) void mfma_experts_kernel(MfmaArgs a)
{
	__shared__ __attribute__((aligned(16))) uint16_t As[2][MT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Bs[2][NT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Alo[SPLIT ? 2 : 1][SPLIT ? MT * LDK : 8];

	const int tile = blockIdx.y;
	if (tile >= *a.ntiles)
		return;
	const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
	const int pbase = a.offsets[e] + m0;
	const int nrows = min(MT, a.offsets[e + 1] - pbase);
	const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
	const int wm = w >> 1, wn = w & 1;
	const int lr = lane & 31, lk = 8 * (lane >> 5);

	// this thread's A row and B source rows/panels
	const int ar = threadIdx.x >> 1;
	const bool alive = ar < nrows;
	const size_t arow_idx = alive ? (DOWN ? (size_t)(pbase + ar) : (size_t)(a.pairs[pbase + ar] / a.k)) : 0;
	const char *arow = SPLIT ? (const char *)(a.a32 + arow_idx * a.in) : (const char *)(a.a16 + arow_idx * a.in);
	const uint8_t *bsrc[2];
	{
		const int bi = (threadIdx.x >> 1) & 63;
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

	const int nk = a.in / KS;
	Pref<TYPE, SPLIT> pf;
	load_step<TYPE, DOWN, SPLIT>(a, bsrc[0], bsrc[1], arow, alive, 0, pf);
	store_step<TYPE, DOWN, SPLIT>(pf, alive, 0, As[0], Alo[0], Bs[0]);
	__syncthreads();
	for (int kk = 0; kk < nk; kk++) {
		const int cur = kk & 1;
		if (kk + 1 < nk)
			load_step<TYPE, DOWN, SPLIT>(a, bsrc[0], bsrc[1], arow, alive, kk + 1, pf);
		const uint16_t *A = As[cur], *B = Bs[cur];
		const uint16_t *AL = Alo[SPLIT ? cur : 0];
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
		if (kk + 1 < nk)
			store_step<TYPE, DOWN, SPLIT>(pf, alive, kk + 1, As[cur ^ 1], Alo[SPLIT ? cur ^ 1 : 0], Bs[cur ^ 1]);
		__syncthreads();
	}

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
