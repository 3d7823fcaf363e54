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

// ------------------------------------------------------------------ B staging
// Thread (m, i, half): panel m (0/1), panel row i, half of the 64-wide K slice.
template <int TYPE>
__device__ __forceinline__ void stage_b(const MfmaArgs &a, int e, int rt0, int kk, uint16_t *__restrict__ Bs)
{
	const int tid = threadIdx.x;
	const int m = tid >> 7, i = (tid >> 1) & 63, h = tid & 1;
	const int nb = a.in / QK;
	uint16_t *dst = Bs + (m * 64 + i) * LDK + 32 * h;
	if (TYPE == TIE_GGML_BF16) {
		// row-major [E][rows][in]; gate/up: matrix m, row rt0*64 + i; down: row (rt0 + m)*64 + i
		const int mat = (a.w[0] == a.w[1]) ? 0 : m;
		const int row = (a.w[0] == a.w[1]) ? (rt0 + m) * 64 + i : rt0 * 64 + i;
		const uint4 *src = reinterpret_cast<const uint4 *>(a.w[mat] + (size_t)e * a.expert_bytes[mat] +
								   ((size_t)row * a.in + kk * KS + 32 * h) * 2);
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<uint4 *>(dst)[c] = src[c];
		return;
	}
	const int b = kk / 4;                  // super-block column
	const int mat = (a.w[0] == a.w[1]) ? 0 : m;
	const int rt = (a.w[0] == a.w[1]) ? rt0 + m : rt0;
	const uint8_t *panel = a.w[mat] + (size_t)e * a.expert_bytes[mat] + ((size_t)rt * nb + b) * panel_bytes(TYPE);
	const uint4 *pc = reinterpret_cast<const uint4 *>(panel) + i;
	float w[32];
	if (TYPE == TIE_GGML_Q4_K) {
		// K slice = group g (sub-blocks 2g, 2g+1); half h = bytes 16h..16h+15 of the group
		const int g = kk & 3;
		const uint4 c0 = pc[0];
		const uint4 q = pc[(1 + 2 * g + h) * 64];
		const float d = half_bits_to_float(c0.x & 0xffffu), dmin = half_bits_to_float(c0.x >> 16);
		const uint32_t s[3] = {c0.y, c0.z, c0.w};
		auto sb = [&](int j) { return (s[j >> 2] >> (8 * (j & 3))) & 0xffu; };
		uint32_t sc0, m0, sc1, m1;
		const int j0 = 2 * g, j1 = 2 * g + 1;
		if (j0 < 4) {
			sc0 = sb(j0) & 63u;
			m0 = sb(j0 + 4) & 63u;
		} else {
			sc0 = (sb(j0 + 4) & 15u) | ((sb(j0 - 4) >> 6) << 4);
			m0 = (sb(j0 + 4) >> 4) | ((sb(j0) >> 6) << 4);
		}
		if (j1 < 4) {
			sc1 = sb(j1) & 63u;
			m1 = sb(j1 + 4) & 63u;
		} else {
			sc1 = (sb(j1 + 4) & 15u) | ((sb(j1 - 4) >> 6) << 4);
			m1 = (sb(j1 + 4) >> 4) | ((sb(j1) >> 6) << 4);
		}
		const float D0 = d * (float)sc0, M0 = -(dmin * (float)m0);
		const float D1 = d * (float)sc1, M1 = -(dmin * (float)m1);
		const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const uint32_t byte = (qw[j >> 2] >> (8 * (j & 3))) & 0xffu;
			w[j] = __builtin_fmaf((float)(byte & 15u), D0, M0);       // K = 16h + j
			w[16 + j] = __builtin_fmaf((float)(byte >> 4), D1, M1);   // K = 32 + 16h + j
		}
		// lo nibbles land at K 16h..16h+15, hi nibbles at 32+16h..: two 16-wide runs
		uint32_t p[16];
#pragma unroll
		for (int j = 0; j < 8; j++) {
			p[j] = pack_bf16(w[2 * j], w[2 * j + 1]);
			p[8 + j] = pack_bf16(w[16 + 2 * j], w[16 + 2 * j + 1]);
		}
		uint16_t *d0 = Bs + (m * 64 + i) * LDK + 16 * h;
		uint16_t *d1 = d0 + 32;
		reinterpret_cast<uint4 *>(d0)[0] = make_uint4(p[0], p[1], p[2], p[3]);
		reinterpret_cast<uint4 *>(d0)[1] = make_uint4(p[4], p[5], p[6], p[7]);
		reinterpret_cast<uint4 *>(d1)[0] = make_uint4(p[8], p[9], p[10], p[11]);
		reinterpret_cast<uint4 *>(d1)[1] = make_uint4(p[12], p[13], p[14], p[15]);
		return;
	} else {
		// Q6_K: K slice = half n of the block, quant rows r = 2*rp + h (elements 32r + l)
		const int n = (kk >> 1) & 1, rp = kk & 1, r = 2 * rp + h;
		const uint4 qa = pc[(4 * n + 2 * (r & 1)) * 64];
		const uint4 qb = pc[(4 * n + 2 * (r & 1) + 1) * 64];
		const uint4 ha = pc[(8 + 2 * n) * 64];
		const uint4 hb = pc[(9 + 2 * n) * 64];
		const uint4 sc = pc[12 * 64];
		const float d = half_bits_to_float(reinterpret_cast<const uint16_t *>(panel + Q6K_CHUNKS * 1024)[i]);
		const uint32_t qlw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
		const uint32_t qhw[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
		const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
		auto scale = [&](int j) { return (float)(int8_t)((scw[j >> 2] >> (8 * (j & 3))) & 0xffu); };
		const float W0 = d * scale(8 * n + 0 + 2 * r), W1 = d * scale(8 * n + 1 + 2 * r);
		const int nsh = 4 * (r >> 1), hsh = 2 * r;
#pragma unroll
		for (int l = 0; l < 32; l++) {
			const uint32_t L = (qlw[l >> 2] >> (8 * (l & 3))) & 0xffu;
			const uint32_t H = (qhw[l >> 2] >> (8 * (l & 3))) & 0xffu;
			const int qv = (int)(((L >> nsh) & 15u) | (((H >> hsh) & 3u) << 4)) - 32;
			w[l] = (l < 16 ? W0 : W1) * (float)qv;
		}
		uint32_t p[16];
#pragma unroll
		for (int j = 0; j < 16; j++)
			p[j] = pack_bf16(w[2 * j], w[2 * j + 1]);
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<uint4 *>(dst)[c] = make_uint4(p[4 * c], p[4 * c + 1], p[4 * c + 2], p[4 * c + 3]);
	}
}

// ------------------------------------------------------------------ A staging
// Thread (row, half): 32 bf16 of the row's 64-wide K slice.  DOWN rows are
// positions in the expert-grouped pair list; gate/up rows are tokens.
template <bool DOWN, bool SPLIT>
__device__ __forceinline__ void stage_a(const MfmaArgs &a, int pbase, int nrows, int kk, uint16_t *__restrict__ As,
					uint16_t *__restrict__ As_lo)
{
	const int tid = threadIdx.x;
	const int r = tid >> 1, h = tid & 1;
	uint16_t *dst = As + r * LDK + 32 * h;
	uint16_t *dlo = SPLIT ? As_lo + r * LDK + 32 * h : nullptr;
	if (r >= nrows) {
#pragma unroll
		for (int c = 0; c < 4; c++) {
			reinterpret_cast<uint4 *>(dst)[c] = make_uint4(0, 0, 0, 0);
			if (SPLIT)
				reinterpret_cast<uint4 *>(dlo)[c] = make_uint4(0, 0, 0, 0);
		}
		return;
	}
	const int p = pbase + r;
	const size_t row = DOWN ? (size_t)p : (size_t)(a.pairs[p] / a.k);
	const size_t col = (size_t)kk * KS + 32 * h;
	if (!SPLIT) {
		const uint4 *src = reinterpret_cast<const uint4 *>(a.a16 + row * a.in + col);
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<uint4 *>(dst)[c] = src[c];
	} else {
		const float4 *src = reinterpret_cast<const float4 *>(a.a32 + row * a.in + col);
#pragma unroll
		for (int c = 0; c < 8; c++) {
			const float4 v = src[c];
			const float hi0 = (float)(__bf16)v.x, hi1 = (float)(__bf16)v.y;
			const float hi2 = (float)(__bf16)v.z, hi3 = (float)(__bf16)v.w;
			reinterpret_cast<uint2 *>(dst)[c] = make_uint2(pack_bf16(hi0, hi1), pack_bf16(hi2, hi3));
			reinterpret_cast<uint2 *>(dlo)[c] =
				make_uint2(pack_bf16(v.x - hi0, v.y - hi1), pack_bf16(v.z - hi2, v.w - hi3));
		}
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
	__shared__ __attribute__((aligned(16))) uint16_t As[MT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Bs[NT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Alo[SPLIT ? MT * LDK : 8];

	const int tile = blockIdx.y;
	if (tile >= *a.ntiles)
		return;
	const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
	const int pbase = a.offsets[e] + m0;
	const int nrows = min(MT, a.offsets[e + 1] - pbase);
	const int rt0 = DOWN ? 2 * blockIdx.x : blockIdx.x; // 64-row panel index of B row 0
	const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
	const int lr = lane & 31, lk = 8 * (lane >> 5);

	f32x16 acc[4];
#pragma unroll
	for (int t = 0; t < 4; t++)
#pragma unroll
		for (int j = 0; j < 16; j++)
			acc[t][j] = 0.0f;

	const int nk = a.in / KS;
	for (int kk = 0; kk < nk; kk++) {
		__syncthreads();
		stage_a<DOWN, SPLIT>(a, pbase, nrows, kk, As, Alo);
		stage_b<TYPE>(a, e, rt0, kk, Bs);
		__syncthreads();
#pragma unroll
		for (int s = 0; s < KS / 16; s++) {
			const bf16x8 av = lds_frag(As, 32 * w + lr, 16 * s + lk);
			bf16x8 alo;
			if (SPLIT)
				alo = lds_frag(Alo, 32 * w + lr, 16 * s + lk);
#pragma unroll
			for (int t = 0; t < 4; t++) {
				const bf16x8 bv = lds_frag(Bs, 32 * t + lr, 16 * s + lk);
				acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc[t], 0, 0, 0);
				if (SPLIT)
					acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo, bv, acc[t], 0, 0, 0);
			}
		}
	}

	// D layout of v_mfma_f32_32x32x16: lane l, register j holds
	// row 8*(j/4) + 4*(l/32) + j%4, column l%32.
#pragma unroll
	for (int j = 0; j < 16; j++) {
		const int mrow = 32 * w + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
		if (mrow >= nrows)
			continue;
		const int p = pbase + mrow;
		if (!DOWN) {
			// acc[0..1]: gate rows 0..63 of the tile, acc[2..3]: the same up rows
#pragma unroll
			for (int t = 0; t < 2; t++) {
				const int col = blockIdx.x * 64 + 32 * t + lr;
				const float hv = tie_swiglu(acc[t][j], acc[t + 2][j], a.silu);
				if (SPLIT)
					a.h32[(size_t)p * a.rows + col] = hv;
				else
					a.h16[(size_t)p * a.rows + col] = bf16_bits(hv);
			}
		} else {
			const int pair = a.pairs[p];
#pragma unroll
			for (int t = 0; t < 4; t++)
				a.y[(size_t)pair * a.rows + rt0 * 64 + 32 * t + lr] = acc[t][j];
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
