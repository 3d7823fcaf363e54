// router.hip -- router logits, top-k selection and softmax gate weights.
//
// Reference: dispatch_mat_vec on ffn_gate_inp (model_qwen3.c:431-432) runs
// mat_vec_row_f32_f32_f32_avx2 (math_avx2.c:228-256): per expert row, 8
// lane accumulators acc[l] += x[8i+l] * w[8i+l] (FMA, i ascending), then
// the hsum_f32_avx2 tree (math_avx2.c:14-21).  find_top_k (engine.c:891-914)
// and softmax over the k selected logits (engine.c:864-888) follow.  The
// kernels below keep those exact operation sequences, so logits, selected
// experts and gate weights are bit-identical to TIE's.
//
// Logit kernels (no cross-workgroup handshakes: an agent-scope fence costs
// more than a launch on this multi-XCD part):
//   router_small   T <= 4: one workgroup per expert row, row and tokens
//                  staged in LDS, one thread per (token, lane) chain.
//   router_mid     up to a few hundred tokens: one workgroup per (expert,
//                  32 tokens), row in LDS, x streamed from L2.
//   router_logits  large T: 32 tokens x 32 experts per workgroup over the
//                  transposed router matrix staged by direct global->LDS
//                  loads.
// Selection kernel: router_topk (a wave per token, E <= 1024).  Small
// batches select
// and group in one workgroup instead (route_group_kernel, dispatch.hip).
#include "common.h"
#include "route.h"

namespace tie {

// Words the next kernels accumulate into (the matrix-core path's per-expert
// pair counts and token masks, and its recomputation count), cleared by
// the logits kernel's workgroups (grid-strided)
__device__ __forceinline__ void zero_words(const ZeroArgs &z)
{
	const int nb = gridDim.x * gridDim.y, b = blockIdx.y * gridDim.x + blockIdx.x;
	for (int i = b * blockDim.x + threadIdx.x; i < z.n; i += nb * blockDim.x)
		z.p[i] = 0;
	for (int i = b * blockDim.x + threadIdx.x; i < z.n2; i += nb * blockDim.x)
		z.p2[i] = 0;
	if (z.one && b == 0 && threadIdx.x == 0)
		*z.one = 0;
}

// ------------------------------------------------------------ router_small
// One token (RS_TOK at most): one workgroup per expert row; the row and the tokens are
// staged in LDS with coalesced 16-byte loads and thread (t, l) runs the
// lane-l chain of token t.  Spreads the 1 MiB router matrix over E
// workgroups, which matters most at T = 1.
constexpr int RS_TOK = 4;
// router_small only for one token: from 2 tokens on router_mid is faster
// (T=4: 11 -> 8.2 us)
#ifndef TIE_RS_MAX_T
#define TIE_RS_MAX_T 1
#endif
constexpr int RS_THREADS = 256;

__global__ __launch_bounds__(RS_THREADS) void router_small_kernel(const float *__restrict__ x,
								  const float *__restrict__ W,
								  const float *__restrict__ bias, int T, int d, int E,
								  float *__restrict__ logits, ZeroArgs z)
{
	zero_words(z);
	extern __shared__ float lds[]; // W row | x [RS_TOK], lane-major (lane_chain)
	float *ws = lds;
	float *xs = lds + lane_major_floats(d);
	const int e = blockIdx.x;
	const int nt = min(RS_TOK, T);
	const int tid = threadIdx.x;

	// the row and the tokens -> LDS, lane-major
	stage_lane_major(ws, W + (size_t)e * d, d);
	for (int t = 0; t < nt; t++)
		stage_lane_major(xs + t * lane_major_floats(d), x + (size_t)t * d, d);
	__syncthreads();
	if (tid >= RS_TOK * 8)
		return;
	const int t = tid >> 3, l = tid & 7;
	const float acc = t < nt ? lane_chain(xs + (size_t)t * lane_major_floats(d), ws, d, l) : 0.0f;
	const float r = hsum8_lanes(acc);
	if (l == 0 && t < nt)
		logits[(size_t)t * E + e] = bias ? r + bias[e] : r;
}

// ------------------------------------------------------------ router_mid
// RS_TOK < T (up to a few hundred tokens): one workgroup per (expert, TOK
// tokens).  The expert row is staged in LDS (read as a broadcast); thread
// (t, l) streams x[t][8i + l] from global memory (L2-resident) with many
// loads in flight and runs the lane-l chain of token t.  TOK tokens per
// workgroup: 16 up to 32 tokens (twice the workgroups, over more CUs),
// else 32.
// U: inputs per lane and batch (d a multiple of 8 U).  LM: the row staged
// lane-major, its weights read a batch ahead in 16-byte reads (263
// registers: one wave per SIMD, so only while one round of workgroups
// covers the grid: up to 64 tokens)
template <int U, int TOK, bool LM>
__global__ __launch_bounds__(TOK * 8) void router_mid_kernel(const float *__restrict__ x,
							     const float *__restrict__ W,
							     const float *__restrict__ bias, int T, int d, int E,
							     float *__restrict__ logits, ZeroArgs z)
{
	zero_words(z);
	extern __shared__ float ws[]; // W row [d]
	const int e = blockIdx.x;
	constexpr int RM_THREADS = TOK * 8;
	const int t0 = blockIdx.y * TOK;
	const int tid = threadIdx.x;
	const int t = t0 + (tid >> 3), l = tid & 7;
	const bool live = t < T;
	const float *xt = x + (size_t)(live ? t : 0) * d + l;
	// the token's inputs stream in batches of U per lane, the next batch
	// loading while the current one is multiplied; the first batch is
	// issued before the row's staging, so the two memory waits overlap
	const int nbt = d / (8 * U);
	float xa[U], xb[U];
#pragma unroll
	for (int u = 0; u < U; u++)
		xa[u] = xt[8 * u];
	float acc = 0.0f;
	if constexpr (LM) {
		// the row lane-major (lane l's weights 8i + l contiguous): one 16-byte
		// LDS read brings 4 steps, and the next batch's weights are read while
		// the current batch is multiplied
		typedef float f4 __attribute__((ext_vector_type(4)));
		stage_lane_major(ws, W + (size_t)e * d, d);
		__syncthreads();
		const f4 *wl = reinterpret_cast<const f4 *>(ws + l * lane_major_stride(d));
		constexpr int U4 = U / 4;
		f4 wa[U4], wb[U4];
#pragma unroll
		for (int q = 0; q < U4; q++)
			wa[q] = wl[q];
		for (int bt = 0; bt < nbt; bt += 2) {
			if (bt + 1 < nbt) {
#pragma unroll
				for (int u = 0; u < U; u++)
					xb[u] = xt[8 * U * (bt + 1) + 8 * u];
#pragma unroll
				for (int q = 0; q < U4; q++)
					wb[q] = wl[U4 * (bt + 1) + q];
			}
#pragma unroll
			for (int u = 0; u < U; u++)
				acc = __builtin_fmaf(xa[u], wa[u / 4][u % 4], acc);
			if (bt + 1 >= nbt)
				break;
			if (bt + 2 < nbt) {
#pragma unroll
				for (int u = 0; u < U; u++)
					xa[u] = xt[8 * U * (bt + 2) + 8 * u];
#pragma unroll
				for (int q = 0; q < U4; q++)
					wa[q] = wl[U4 * (bt + 2) + q];
			}
#pragma unroll
			for (int u = 0; u < U; u++)
				acc = __builtin_fmaf(xb[u], wb[u / 4][u % 4], acc);
	}
	} else {
		const float4 *W4 = reinterpret_cast<const float4 *>(W + (size_t)e * d);
		for (int i = tid; i < (d >> 2); i += RM_THREADS)
			reinterpret_cast<float4 *>(ws)[i] = W4[i];
		__syncthreads();
		const float *wl = ws + l;
		for (int bt = 0; bt < nbt; bt += 2) {
			if (bt + 1 < nbt) {
#pragma unroll
				for (int u = 0; u < U; u++)
					xb[u] = xt[8 * U * (bt + 1) + 8 * u];
			}
#pragma unroll
			for (int u = 0; u < U; u++)
				acc = __builtin_fmaf(xa[u], wl[8 * U * bt + 8 * u], acc);
			if (bt + 1 >= nbt)
				break;
			if (bt + 2 < nbt) {
#pragma unroll
				for (int u = 0; u < U; u++)
					xa[u] = xt[8 * U * (bt + 2) + 8 * u];
			}
#pragma unroll
			for (int u = 0; u < U; u++)
				acc = __builtin_fmaf(xb[u], wl[8 * U * (bt + 1) + 8 * u], acc);
	}
	}
	const float r = hsum8_lanes(acc);
	if (l == 0 && live)
		logits[(size_t)t * E + e] = bias ? r + bias[e] : r;
}

// ------------------------------------------------------------ router_logits
// One workgroup (8 waves) per RT_TOK tokens x 32 experts.  Thread (l, eg,
// tg) runs the lane-l chains of experts 4eg..4eg+3 x tokens RT_TPT*tg..,
// each in TIE's order (i ascending): per step one 16-byte LDS read of the 4
// weights and RT_TPT reads of x feed 4*RT_TPT FMAs.  K advances RT_KC at a
// time through a double-buffered LDS pipeline filled by direct global->LDS
// loads (global_load_lds_dwordx4): the x rows as they are (token-major) and
// the matching RT_KC rows x 32 experts of the transposed router matrix,
// whose 16-byte column groups are XOR-swizzled by row (conflict-free
// reads).  16 tokens and 128-wide K chunks keep the LDS at 48 KiB (three
// workgroups per CU); 32 x 256 (128 KiB, one per CU) took 33 us at T = 512
// against 26 us.
#ifndef TIE_RT_TOK
#define TIE_RT_TOK 16
#endif
#ifndef TIE_RT_KC
#define TIE_RT_KC 128
#endif
constexpr int RT_TOK = TIE_RT_TOK, RT_EXP = 32, RT_KC = TIE_RT_KC, RT_THREADS = 512, RT_NW = RT_THREADS / 64;
constexpr int RT_TPT = RT_TOK / 8;              // tokens per thread
constexpr int RT_WBYTES = RT_KC * RT_EXP * 4;   // W^T chunk (16 KiB)
constexpr int RT_XBYTES = RT_TOK * RT_KC * 4;   // x chunk (8 KiB)
constexpr int RT_BUF = RT_WBYTES + RT_XBYTES;
constexpr int RT_LDS = 2 * RT_BUF;              // double-buffered (48 KiB: three workgroups per CU)
#ifndef TIE_RT_IB
#define TIE_RT_IB 16
#endif
constexpr int RT_IB = TIE_RT_IB < RT_KC / 8 ? TIE_RT_IB : RT_KC / 8; // K steps whose operands are read ahead
// the tiled kernel above this many tokens (below: router_mid)
#ifndef TIE_RT_MIN_T
#define TIE_RT_MIN_T 256
#endif

// The LDS offset of a generic pointer into LDS: a flat LDS address is the
// shared aperture's base in the high 32 bits and the offset in the low 32,
// so truncation gives the offset (a cast to the LDS address space would add
// a null-pointer test: a 64-bit compare and select per address).
__device__ __forceinline__ uint32_t rt_lds_addr(const void *p)
{
	return (uint32_t)(uintptr_t)p;
}

// 16 bytes from global memory to LDS address lds + 16 * lane (inline asm:
// the stage barrier, not the compiler, waits for it)
__device__ __forceinline__ void rt_dma16(const void *g, uint32_t lds)
{
	asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// chunk kc of W^T (8 rows per wave instruction; slot s of row r holds
// column group s ^ (r%8)) and of x (one 1 KiB token row per instruction)
__device__ __forceinline__ void rt_dma_chunk(const float *__restrict__ x, const float *__restrict__ WT, int E, int d,
					     int t0, int e0, int nt, int kc, uint8_t *buf)
{
	const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
	for (int c = 0; c < RT_KC / 8 / RT_NW; c++) {
		const int row0 = 8 * (RT_NW * c + w), row = row0 + (lane >> 3);
		const int cg = (lane & 7) ^ (row & 7);
		rt_dma16(WT + (size_t)(kc + row) * E + e0 + 4 * cg,
			 __builtin_amdgcn_readfirstlane(rt_lds_addr(buf + row0 * RT_EXP * 4)));
	}
#pragma unroll
	for (int c = 0; c < RT_TOK / RT_NW; c++) {
		const int t = RT_NW * c + w;
		if (t < nt && lane < RT_KC / 4)
			rt_dma16(x + (size_t)(t0 + t) * d + kc + 4 * lane,
				 __builtin_amdgcn_readfirstlane(rt_lds_addr(buf + RT_WBYTES + t * RT_KC * 4)));
	}
}

__device__ __forceinline__ void rt_barrier()
{
	asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef _Float16 rt_f16x8 __attribute__((ext_vector_type(8)));

// XConvArgs' conversion of the RT_TOK x RT_KC chunk staged at xs (token-major
// rows of RT_KC floats), K offset kc: thread (t, q) of the first 16 RT_TOK
// converts floats 8q .. 8q + 7 of token t; bad: its range flag so far
__device__ __forceinline__ void rt_convert_chunk(const float *xs, const XConvArgs &xc, int t0, int nt, int d, int kc,
						 int &bad)
{
	constexpr int QPT = RT_KC / 8; // threads per token
	const int t = threadIdx.x / QPT, q = threadIdx.x % QPT;
	if (t >= nt || threadIdx.x >= RT_TOK * QPT)
		return;
	const float4 a = *reinterpret_cast<const float4 *>(xs + t * RT_KC + 8 * q);
	const float4 c = *reinterpret_cast<const float4 *>(xs + t * RT_KC + 8 * q + 4);
	const float m = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(a.x), __builtin_fabsf(a.y)),
							__builtin_fmaxf(__builtin_fabsf(a.z), __builtin_fabsf(a.w))),
					__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(c.x), __builtin_fabsf(c.y)),
							__builtin_fmaxf(__builtin_fabsf(c.z), __builtin_fabsf(c.w))));
	// fmax drops NaN: test the values themselves for NaN
	const bool nan = a.x != a.x || a.y != a.y || a.z != a.z || a.w != a.w || c.x != c.x || c.y != c.y ||
			 c.z != c.z || c.w != c.w;
	bad |= (nan || !(m < 65504.0f)) ? 1 : 0;
	const rt_f16x8 h = {(_Float16)a.x, (_Float16)a.z, (_Float16)a.y, (_Float16)a.w,
			    (_Float16)c.x, (_Float16)c.z, (_Float16)c.y, (_Float16)c.w};
	*reinterpret_cast<rt_f16x8 *>(xc.xa + (size_t)(t0 + t) * d + kc + 8 * q) = h;
}

__global__ __launch_bounds__(RT_THREADS) void router_logits_kernel(const float *__restrict__ x,
								   const float *__restrict__ WT,
								   const float *__restrict__ bias, int T, int d, int E,
								   float *__restrict__ logits, ZeroArgs z, XConvArgs xc)
{
	zero_words(z);
	extern __shared__ __attribute__((aligned(16))) uint8_t rt_lds[];

	const int tid = threadIdx.x;
	const int l = tid & 7, eg = (tid >> 3) & 7, tg = tid >> 6;
	const int t0 = blockIdx.x * RT_TOK, e0 = blockIdx.y * RT_EXP;
	const int nt = min(RT_TOK, T - t0);
	const int nkc = d / RT_KC;
	// float index of experts 4eg.. in W^T row r: slot eg ^ (r%8), r % 8 == l
	const int wcol = 4 * (eg ^ l);
	const int xo = (RT_TPT * tg) * RT_KC + l;

	float acc[RT_TPT][4];
#pragma unroll
	for (int a = 0; a < RT_TPT; a++)
#pragma unroll
		for (int b = 0; b < 4; b++)
			acc[a][b] = 0.0f;

	// the first expert tile's workgroups also convert their tokens' x rows
	const bool conv = xc.xa && blockIdx.y == 0;
	int bad = 0;

	rt_dma_chunk(x, WT, E, d, t0, e0, nt, 0, rt_lds);
	rt_barrier();
	for (int c = 0; c < nkc; c++) {
		if (c + 1 < nkc)
			rt_dma_chunk(x, WT, E, d, t0, e0, nt, (c + 1) * RT_KC, rt_lds + ((c + 1) & 1) * RT_BUF);
		const float *ws = reinterpret_cast<const float *>(rt_lds + (c & 1) * RT_BUF);
		const float *xs = reinterpret_cast<const float *>(rt_lds + (c & 1) * RT_BUF + RT_WBYTES);
		// before the FMAs: the stores have the chunk's FMAs to land before the
		// stage barrier (which waits for every vector memory operation)
		if (conv)
			rt_convert_chunk(xs, xc, t0, nt, d, c * RT_KC, bad);
		// operands of RT_IB K steps read into registers first (their LDS
		// latencies overlap), then the FMAs in K order
		for (int i0 = 0; i0 < RT_KC / 8; i0 += RT_IB) {
			float4 w4[RT_IB];
			float xv[RT_IB][RT_TPT];
#pragma unroll
			for (int j = 0; j < RT_IB; j++) {
				w4[j] = *reinterpret_cast<const float4 *>(ws + (8 * (i0 + j) + l) * RT_EXP + wcol);
#pragma unroll
				for (int a = 0; a < RT_TPT; a++)
					xv[j][a] = xs[xo + a * RT_KC + 8 * (i0 + j)];
			}
#pragma unroll
			for (int j = 0; j < RT_IB; j++) {
#pragma unroll
				for (int a = 0; a < RT_TPT; a++) {
					acc[a][0] = __builtin_fmaf(xv[j][a], w4[j].x, acc[a][0]);
					acc[a][1] = __builtin_fmaf(xv[j][a], w4[j].y, acc[a][1]);
					acc[a][2] = __builtin_fmaf(xv[j][a], w4[j].z, acc[a][2]);
					acc[a][3] = __builtin_fmaf(xv[j][a], w4[j].w, acc[a][3]);
				}
			}
		}
		rt_barrier();
	}
	if (conv) {
		// a token's flag: the OR over its RT_KC / 8 threads (aligned lane groups)
		constexpr int QPT = RT_KC / 8;
		static_assert(64 % QPT == 0, "a token's threads in one wave");
		const unsigned long long b = __ballot(bad);
		const int lane = tid & 63, t = tid / QPT;
		if (tid < RT_TOK * QPT && lane % QPT == 0 && t < nt)
			xc.flag[t0 + t] = ((b >> lane) & ((1ull << QPT) - 1ull)) != 0 ? 1 : 0;
	}

	// hsum8 over the 8 lanes l of each chain group (math_avx2.c:14-21 order)
#pragma unroll
	for (int a = 0; a < RT_TPT; a++) {
#pragma unroll
		for (int b = 0; b < 4; b++) {
			float r = hsum8_lanes(acc[a][b]);
			const int t = RT_TPT * tg + a, e = e0 + 4 * eg + b;
			if (l == 0 && t < nt) {
				if (bias)
					r = r + bias[e];
				logits[(size_t)(t0 + t) * E + e] = r;
			}
		}
	}
}

// W [E][d] -> W^T [d][E] (once, at layer creation)
__global__ void transpose_kernel(const float *__restrict__ W, float *__restrict__ WT, int E, int d)
{
	__shared__ float tile[32][33];
	const int bx = blockIdx.x * 32, by = blockIdx.y * 32; // bx: k, by: e
	for (int i = threadIdx.y; i < 32; i += 8) {
		const int e = by + i, kk = bx + threadIdx.x;
		tile[i][threadIdx.x] = (e < E && kk < d) ? W[(size_t)e * d + kk] : 0.0f;
	}
	__syncthreads();
	for (int i = threadIdx.y; i < 32; i += 8) {
		const int kk = bx + i, e = by + threadIdx.x;
		if (kk < d && e < E)
			WT[(size_t)kk * E + e] = tile[threadIdx.x][i];
	}
}

hipError_t launch_router_transpose(const Layer &L, hipStream_t s)
{
	tie_launch(transpose_kernel, dim3((L.d + 31) / 32, (L.E + 31) / 32), dim3(32, 8), 0, s, L.router,
			   (float *)L.routerT, L.E, L.d);
	return hipGetLastError();
}

// ------------------------------------------------------------ router_topk
// one wave per token (topk_softmax, E <= MAX_E)
constexpr int RW_THREADS = 256;
__global__ __launch_bounds__(RW_THREADS) void router_topk_kernel(const float *__restrict__ logits, int T, int E,
								      int k, int32_t *__restrict__ topk_idx,
								      float *__restrict__ topk_w, int routing,
								      const float *__restrict__ pbias)
{
	__shared__ uint64_t etab[32];
	if (threadIdx.x < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		etab[threadIdx.x] = tab[threadIdx.x];
	}
	__syncthreads();
	const int t = blockIdx.x * (RW_THREADS / 64) + (threadIdx.x >> 6);
	if (t < T)
		topk_softmax(logits + (size_t)t * E, E, k, etab, topk_idx + (size_t)t * k, topk_w + (size_t)t * k, routing,
			     pbias);
}

static bool router_tiled(const Layer &L, int T)
{
	return T > TIE_RT_MIN_T && L.E % RT_EXP == 0 && L.d % RT_KC == 0 && L.routerT;
}

bool router_converts_x(const Layer &L, int T)
{
	return router_tiled(L, T);
}

hipError_t launch_router_logits(const Layer &L, const float *x, int T, float *logits, hipStream_t s, ZeroArgs z,
				XConvArgs xc)
{
	const int d = L.d, E = L.E;
	if (T <= TIE_RS_MAX_T && sizeof(float) * (size_t)(8 * (d / 8 + 4)) * (1 + RS_TOK) <= 160 * 1024) {
		const size_t lds = sizeof(float) * (size_t)(8 * (d / 8 + 4)) * (1 + RS_TOK);
		tie_launch(router_small_kernel, dim3(E), dim3(RS_THREADS), lds, s, x, L.router, L.bias, T, d, E,
				   logits, z);
		return hipGetLastError();
	}
	// the tiled kernel above 256 tokens: below that its one chunk in flight
	// per K step leaves it waiting on memory, and router_mid is faster
	if (router_tiled(L, T)) {
		static bool attr = false;
		if (!attr) {
			const hipError_t err = hipFuncSetAttribute((const void *)router_logits_kernel,
								   hipFuncAttributeMaxDynamicSharedMemorySize, RT_LDS);
			if (err != hipSuccess)
				return err;
			attr = true;
		}
		tie_launch(router_logits_kernel, dim3((T + RT_TOK - 1) / RT_TOK, E / RT_EXP), dim3(RT_THREADS),
				   RT_LDS, s, x, L.routerT, L.bias, T, d, E, logits, z, xc);
		return hipGetLastError();
	}
	const bool u64 = d % 512 == 0;
	const int tok = T <= 32 ? 16 : 32;
	const bool lm = T <= 64;
	auto kern = lm ? (tok == 16 ? (u64 ? router_mid_kernel<64, 16, true> : router_mid_kernel<32, 16, true>)
				    : (u64 ? router_mid_kernel<64, 32, true> : router_mid_kernel<32, 32, true>))
		       : (u64 ? router_mid_kernel<64, 32, false> : router_mid_kernel<32, 32, false>);
	tie_launch(kern, dim3(E, (T + tok - 1) / tok), dim3(tok * 8),
			   sizeof(float) * (size_t)(lm ? lane_major_floats(d) : d), s, x, L.router, L.bias, T, d, E, logits, z);
	return hipGetLastError();
}

hipError_t launch_router_select(const Layer &L, int T, int k, const float *logits, int32_t *topk_idx, float *topk_w,
				hipStream_t s)
{
	tie_launch(router_topk_kernel, dim3((T + RW_THREADS / 64 - 1) / (RW_THREADS / 64)), dim3(RW_THREADS), 0,
			   s, logits, T, L.E, k, topk_idx, topk_w, L.routing, L.pbias);
	return hipGetLastError();
}

hipError_t launch_router(const Layer &L, const float *x, int T, int k, float *logits, int32_t *topk_idx,
			 float *topk_w, hipStream_t s)
{
	hipError_t err = launch_router_logits(L, x, T, logits, s);
	if (err != hipSuccess)
		return err;
	return launch_router_select(L, T, k, logits, topk_idx, topk_w, s);
}

} // namespace tie
