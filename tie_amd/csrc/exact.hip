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
// Work decomposition (pairs = (token, slot) grouped by expert by
// dispatch.hip):
//   exact_q_rows    one workgroup per (64-row tile, active expert, matrix);
//                   wave w owns block column w, lane i owns row i of the
//                   tile.  The lane's super-block (144 or 210 bytes) is
//                   read from the panel layout with coalesced 16-byte loads
//                   and kept in VGPRs for every token routed to the expert;
//                   the token's input vector is staged in LDS and read as
//                   wave-uniform broadcasts; per-block dots meet in LDS and
//                   lane i of wave 0 adds them in block order.
//   exact_bf16_rows two threads per row, each owning four of the row's
//                   eight lane accumulators.
// Gate and up write their row sums; the down kernel applies TIE's table
// SwiGLU while staging its input vector, so no separate activation pass.
#include "common.h"

namespace tie {

// Input vectors (x for gate/up, the SwiGLU output h for down) are read
// through the constant address space: every lane of a wave reads the same
// address, so the loads become scalar (s_load) and the values reach the
// FMAs as SGPR operands -- no LDS staging, no broadcast traffic.
typedef const float __attribute__((address_space(4))) cfloat;

// The launders below are empty asm statements that make a value opaque to
// the compiler at one point of the instruction stream.  Without them the
// scheduler hoists all 256 dequantised weights or all 256 input values of
// a super-block to the top of the dot product and runs out of registers.
__device__ __forceinline__ void launder(cfloat *&p)
{
	asm volatile("" : "+s"(p));
}

// ------------------------------------------------------------------ blocks
struct Q4KBlock {
	uint4 c[Q4K_CHUNKS];
};
struct Q6KBlock {
	uint4 c[Q6K_CHUNKS];
	uint32_t d;
};

__device__ __forceinline__ void load_block(const uint8_t *__restrict__ panel, int lane, Q4KBlock &B)
{
	const uint4 *p = reinterpret_cast<const uint4 *>(panel) + lane;
#pragma unroll
	for (int c = 0; c < Q4K_CHUNKS; c++)
		B.c[c] = p[c * 64];
}

__device__ __forceinline__ void load_block(const uint8_t *__restrict__ panel, int lane, Q6KBlock &B)
{
	const uint4 *p = reinterpret_cast<const uint4 *>(panel) + lane;
#pragma unroll
	for (int c = 0; c < Q6K_CHUNKS; c++)
		B.c[c] = p[c * 64];
	B.d = reinterpret_cast<const uint16_t *>(panel + Q6K_CHUNKS * 1024)[lane];
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int i)
{
	return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ float ubyte(uint32_t w, int i)
{
	return (float)((w >> (8 * i)) & 0xffu);
}

// dot_product_f32_q4k_avx2 (math_avx2.c:535-604) for the lane's block.
template <typename XP>
__device__ __forceinline__ float block_dot(const Q4KBlock &B, XP *x)
{
	const uint32_t w0 = B.c[0].x;
	const float d = half_bits_to_float(w0 & 0xffffu);
	const float dmin = half_bits_to_float(w0 >> 16);
	const uint32_t s[3] = {B.c[0].y, B.c[0].z, B.c[0].w}; // 12 packed scale/min bytes
	float D[8], nM[8];
#pragma unroll
	for (int j = 0; j < 8; j++) {
		auto sb = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
		uint32_t sc, m;
		if (j < 4) {
			sc = sb(j) & 63u;
			m = sb(j + 4) & 63u;
		} else {
			sc = (sb(j + 4) & 15u) | ((sb(j - 4) >> 6) << 4);
			m = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
		}
		D[j] = d * (float)sc;
		nM[j] = -(dmin * (float)m);
	}
	float a0[8], a1[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		a0[l] = a1[l] = 0.0f;
#pragma unroll
	for (int g = 0; g < 4; g++) {
		const float D1 = D[2 * g], M1 = nM[2 * g], D2 = D[2 * g + 1], M2 = nM[2 * g + 1];
#pragma unroll
		for (int o = 0; o < 2; o++) {
			uint4 q = B.c[1 + 2 * g + o];
			asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w)::"memory");
			XP *xl = x + 64 * g + 16 * o;
			launder(xl);
			XP *xh = xl + 32;
#pragma unroll
			for (int h = 0; h < 4; h++) {
				const uint32_t w = word(q, h);
				uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
				asm volatile("" : "+v"(lo), "+v"(hi)); // keeps one mask per 4 bytes + v_cvt_f32_ubyteN
#pragma unroll
				for (int i = 0; i < 4; i++) {
					const int m = 4 * h + i;
					float &A = (m < 8) ? a0[m & 7] : a1[m & 7];
					A = __builtin_fmaf(xl[m], __builtin_fmaf(ubyte(lo, i), D1, M1), A);
					A = __builtin_fmaf(xh[m], __builtin_fmaf(ubyte(hi, i), D2, M2), A);
				}
			}
		}
	}
	float v[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		v[l] = a0[l] + a1[l];
	return hsum8(v);
}

// dot_product_f32_q6k_avx2 (math_avx2.c:411-495) for the lane's block.
// Panel chunks: 0-7 ql[0..127], 8-11 qh[0..63], 12 the int8 scales.
template <typename XP>
__device__ __forceinline__ float block_dot(const Q6KBlock &B, XP *x)
{
	const float d = half_bits_to_float(B.d);
	float a0[8], a1[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		a0[l] = a1[l] = 0.0f;
#pragma unroll
	for (int n = 0; n < 2; n++) {
#pragma unroll
		for (int l = 0; l < 32; l += 8) {
			const int is = (l >= 16) ? 1 : 0;
			auto sc = [&](int j) {
				return (float)(int8_t)((word(B.c[12], j >> 2) >> (8 * (j & 3))) & 0xffu);
			};
			const float W0 = d * sc(8 * n + is + 0);
			const float W1 = d * sc(8 * n + is + 2);
			const float W2 = d * sc(8 * n + is + 4);
			const float W3 = d * sc(8 * n + is + 6);
			const uint4 &cl = B.c[4 * n + (l >> 4)];
			const uint4 &cl2 = B.c[4 * n + 2 + (l >> 4)];
			const uint4 &chh = B.c[8 + 2 * n + (l >> 4)];
#pragma unroll
			for (int hw = 0; hw < 2; hw++) {
					const int dw = ((l & 8) >> 2) + hw;
				uint32_t L = word(cl, dw), L2 = word(cl2, dw), H = word(chh, dw);
				asm volatile("" : "+v"(L), "+v"(L2), "+v"(H)::"memory");
				XP *xq = x + 128 * n + l + 4 * hw;
				launder(xq);
				const uint32_t q1 = (L & 0x0f0f0f0fu) | ((H & 0x03030303u) << 4);
				const uint32_t q2 = (L2 & 0x0f0f0f0fu) | (((H >> 2) & 0x03030303u) << 4);
				const uint32_t q3 = ((L >> 4) & 0x0f0f0f0fu) | (((H >> 4) & 0x03030303u) << 4);
				const uint32_t q4 = ((L2 >> 4) & 0x0f0f0f0fu) | (((H >> 6) & 0x03030303u) << 4);
#pragma unroll
				for (int i = 0; i < 4; i++) {
					const int m = 4 * hw + i;
					XP *xb = xq + i;
					a0[m] = __builtin_fmaf(W0, (ubyte(q1, i) - 32.0f) * xb[0], a0[m]);
					a1[m] = __builtin_fmaf(W1, (ubyte(q2, i) - 32.0f) * xb[32], a1[m]);
					a0[m] = __builtin_fmaf(W2, (ubyte(q3, i) - 32.0f) * xb[64], a0[m]);
					a1[m] = __builtin_fmaf(W3, (ubyte(q4, i) - 32.0f) * xb[96], a1[m]);
				}
			}
		}
	}
	float v[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		v[l] = a0[l] + a1[l];
	return hsum8(v);
}

template <int TYPE> struct BlockOf;
template <> struct BlockOf<TIE_GGML_Q4_K> {
	using type = Q4KBlock;
};
template <> struct BlockOf<TIE_GGML_Q6_K> {
	using type = Q6KBlock;
};

struct RowsArgs {
	const uint8_t *w[2];  // expert tensor data (panel layout / BF16 row-major)
	float *sums[2];       // [pairs][rows] row results (gate, up) or y (down)
	size_t expert_bytes[2];
	int rows, in, k, E;
	const float *x;       // [T][in] (gate/up) or h [pairs][in] (down)
	float *h;             // [pairs][rows] SwiGLU output (gate/up)
	uint32_t *tile_cnt;   // [pairs][rows/64] gate/up completion counters
	const float *silu;
	const int32_t *offsets, *pairs, *active;
	int mat_base;         // matrix index of blockIdx.z == 0 (0 gate, 1 up)
};

// Gate/up completion: each (pair, 64-row tile) is finished by two
// workgroups, the gate one and the up one.  Both publish their row sums;
// the second to arrive (counter 0 -> 1 -> reset) applies TIE's table SwiGLU
// (swiglu_activation_f32_f32_avx2) to the tile and writes h.
__device__ __forceinline__ void finish_gate_up(const RowsArgs &a, int m, int pair, int rt, int lane, float s)
{
	const int nrt = a.rows / PANEL_ROWS;
	const size_t o = (size_t)pair * a.rows + rt * PANEL_ROWS + lane;
	a.sums[m][o] = s;
	__threadfence();
	uint32_t prev = 0;
	uint32_t *cnt = a.tile_cnt + (size_t)pair * nrt + rt;
	if (lane == 0)
		prev = atomicAdd(cnt, 1u);
	prev = __shfl(prev, 0);
	if (prev == 1) {
		__threadfence();
		const float other = __hip_atomic_load(a.sums[1 - m] + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		const float g = m == 0 ? s : other;
		const float u = m == 0 ? other : s;
		a.h[o] = tie_swiglu(g, u, a.silu);
		if (lane == 0)
			__hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
	}
}

// ------------------------------------------------------------ exact_q_rows
// One workgroup per (64-row tile, active expert, matrix).  Wave w owns
// super-block columns w, w + 8, ...; lane i owns row i of the tile.  Per
// pair the lane loads its block (coalesced panel chunks), forms the block
// dot with the pair's input vector read by scalar loads, and the per-block
// dots meet in LDS where wave 0 adds them in block order.
constexpr int MAX_NB = 64; // super-blocks per row (in <= 16384)
constexpr int Q_WAVES = 8;

template <int TYPE, bool DOWN>
__global__ __launch_bounds__(64 * Q_WAVES) void exact_q_rows_kernel(RowsArgs a)
{
	using Block = typename BlockOf<TYPE>::type;
	__shared__ float part[MAX_NB][64];
	const int m = a.mat_base + blockIdx.z;
	const int slot = blockIdx.y;
	if (slot >= a.active[a.E])
		return;
	const int e = a.active[slot];
	const int p0 = a.offsets[e], p1 = a.offsets[e + 1];
	const int rt = blockIdx.x;
	const int lane = threadIdx.x & 63;
	const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int nw = blockDim.x >> 6;
	const int nb = a.in / QK;
	const size_t pb = panel_bytes(TYPE);
	const uint8_t *panels = a.w[m] + (size_t)e * a.expert_bytes[m] + (size_t)rt * nb * pb;

	for (int p = p0; p < p1; p++) {
		const int pair = __builtin_amdgcn_readfirstlane(a.pairs[p]);
		cfloat *xin = (cfloat *)(DOWN ? a.x + (size_t)pair * a.in : a.x + (size_t)(pair / a.k) * a.in);
		for (int b = w; b < nb; b += nw) {
			Block blk;
			load_block(panels + (size_t)b * pb, lane, blk);
			part[b][lane] = block_dot(blk, xin + QK * b);
		}
		__syncthreads();
		if (w == 0) {
			float s = 0.0f; // serial sum over super-blocks (math_avx2.c:762-766)
			for (int b = 0; b < nb; b++)
				s = s + part[b][lane];
			if (DOWN)
				a.sums[m][(size_t)pair * a.rows + rt * PANEL_ROWS + lane] = s;
			else
				finish_gate_up(a, m, pair, rt, lane, s);
		}
		__syncthreads();
	}
}

// --------------------------------------------------------- exact_bf16_rows
// mat_vec_row_f32_bf16_f32_avx2 + dot_product_f32_bf16_avx2
// (math_avx2.c:148-158, 188-226): 8 lane accumulators over the whole row,
// then hsum8.  Thread h of a row owns lanes 4h..4h+3; a workgroup covers
// 64 rows (128 threads) so gate/up tiles match the SwiGLU completion tiles.
template <bool DOWN>
__global__ __launch_bounds__(128) void exact_bf16_rows_kernel(RowsArgs a)
{
	const int m = a.mat_base + blockIdx.z;
	const int slot = blockIdx.y;
	if (slot >= a.active[a.E])
		return;
	const int e = a.active[slot];
	const int p0 = a.offsets[e], p1 = a.offsets[e + 1];
	const int rt = blockIdx.x;
	const int r = threadIdx.x >> 1; // row within the tile
	const int h = threadIdx.x & 1;
	const int row = rt * PANEL_ROWS + r;
	const uint16_t *wr = reinterpret_cast<const uint16_t *>(a.w[m] + (size_t)e * a.expert_bytes[m]) +
			     (size_t)row * a.in;

	for (int p = p0; p < p1; p++) {
		const int pair = a.pairs[p];
		const float *xin = DOWN ? a.x + (size_t)pair * a.in : a.x + (size_t)(pair / a.k) * a.in;
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
		const float s = (s0 + s1) + (s2 + s3);
		// rows of this tile gathered onto wave 0 lanes 0..63 through LDS
		__shared__ float rs[PANEL_ROWS];
		if (h == 0)
			rs[r] = s;
		__syncthreads();
		if (threadIdx.x < 64) {
			const float v = rs[threadIdx.x];
			if (DOWN)
				a.sums[m][(size_t)pair * a.rows + rt * PANEL_ROWS + threadIdx.x] = v;
			else
				finish_gate_up(a, m, pair, rt, threadIdx.x, v);
		}
		__syncthreads();
	}
}

// ---------------------------------------------------------------- launcher
template <bool DOWN>
static hipError_t launch_rows(const Layer &L, int mat_base, int nmat, const ExpertTensor &t, int k, int max_active,
			      const float *x, Workspace &ws, const float *silu, int npairs, hipStream_t s)
{
	RowsArgs a;
	if (DOWN) {
		a.w[0] = a.w[1] = L.down.data;
		a.expert_bytes[0] = a.expert_bytes[1] = L.down.expert_bytes;
		a.sums[0] = a.sums[1] = ws.y;
	} else {
		a.w[0] = L.gate.data;
		a.w[1] = L.up.data;
		a.expert_bytes[0] = L.gate.expert_bytes;
		a.expert_bytes[1] = L.up.expert_bytes;
		a.sums[0] = ws.h + (size_t)npairs * L.F;     // gate sums
		a.sums[1] = ws.h + 2 * (size_t)npairs * L.F; // up sums
	}
	a.rows = t.rows;
	a.in = t.in;
	a.k = k;
	a.E = L.E;
	a.x = x;
	a.h = ws.h;
	a.tile_cnt = ws.tile_cnt;
	a.silu = silu;
	a.offsets = ws.offsets;
	a.pairs = ws.pairs;
	a.active = ws.active;
	a.mat_base = mat_base;
	dim3 grid(t.rows / PANEL_ROWS, max_active, nmat);
	if (t.type == TIE_GGML_BF16) {
		hipLaunchKernelGGL(exact_bf16_rows_kernel<DOWN>, grid, dim3(128), 0, s, a);
	} else {
		const int nb = t.in / QK;
		const int waves = nb < Q_WAVES ? nb : Q_WAVES;
		if (t.type == TIE_GGML_Q4_K)
			hipLaunchKernelGGL((exact_q_rows_kernel<TIE_GGML_Q4_K, DOWN>), grid, dim3(64 * waves), 0, s, a);
		else
			hipLaunchKernelGGL((exact_q_rows_kernel<TIE_GGML_Q6_K, DOWN>), grid, dim3(64 * waves), 0, s, a);
	}
	return hipGetLastError();
}

// ws.h holds three [pairs][F] planes: h (SwiGLU output), gate sums, up sums.
hipError_t launch_exact_experts(const Layer &L, const float *x, int T, int k, const float *silu, Workspace &ws,
				hipStream_t s)
{
	const int npairs = T * k;
	const int max_active = npairs < L.E ? npairs : L.E;
	if (npairs == 0)
		return hipSuccess;
	hipError_t err;
	prof_begin("exact_gate_up", s);
	if (L.gate.type == L.up.type)
		err = launch_rows<false>(L, 0, 2, L.gate, k, max_active, x, ws, silu, npairs, s);
	else {
		err = launch_rows<false>(L, 0, 1, L.gate, k, max_active, x, ws, silu, npairs, s);
		if (err == hipSuccess)
			err = launch_rows<false>(L, 1, 1, L.up, k, max_active, x, ws, silu, npairs, s);
	}
	prof_end(s);
	if (err != hipSuccess)
		return err;
	prof_begin("exact_down", s);
	err = launch_rows<true>(L, 0, 1, L.down, k, max_active, ws.h, ws, silu, npairs, s);
	prof_end(s);
	return err;
}

} // namespace tie
