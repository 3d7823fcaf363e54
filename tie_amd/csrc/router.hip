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
// Two shapes:
//   router_small   one workgroup per (expert, group of 4 tokens); the expert
//                  row and the tokens are staged in LDS with coalesced
//                  16-byte loads, one thread per (token, lane) runs the
//                  256-long FMA chain.  Used for small T, where spreading the
//                  1 MiB router matrix over E workgroups matters most.  The
//                  last workgroup of a token group (completion counter,
//                  self-resetting) does top-k + softmax for its tokens.
//   router_logits  one workgroup per 32 tokens x 32 experts over the
//   + router_topk  transposed router matrix (stored at layer creation);
//                  each thread runs 16 independent lane chains from LDS
//                  tiles.  A second kernel selects the experts, 8 lanes per
//                  token: no cross-workgroup handshake, whose agent-scope
//                  fences cost more than the launch on this multi-XCD part.
#include "common.h"
#include "tie_expf.h"

namespace tie {

// top-k (engine.c:891-914 semantics) + softmax (engine.c:864-888) for one
// token, by one wave.  `lg` holds the token's E logits.  The k winners are
// extracted one at a time by a wave-wide argmax under the order (value
// descending, index ascending) -- the order find_top_k's strict-greater
// insertion produces; NaN and -inf never qualify; unfilled slots are
// {-1, -inf}.  Slot j's exponential is computed by lane j, the sum is
// formed serially in slot order, and every weight is e_j * (1 / sum).
__device__ void topk_softmax_wave(const float *lg, int E, int k, const uint64_t *etab, int32_t *out_idx,
				  float *out_w)
{
	const int lane = threadIdx.x & 63;
	constexpr int PER = MAX_E / 64;
	float v[PER];
#pragma unroll
	for (int q = 0; q < PER; q++) {
		const int e = q * 64 + lane;
		const float x = e < E ? lg[e] : -__builtin_inff();
		v[q] = (x > -__builtin_inff()) ? x : -__builtin_inff(); // NaN -> never selected
	}
	float my_s = -__builtin_inff();
	int my_i = -1;
	for (int j = 0; j < k; j++) {
		// lane-local best: first (lowest index) maximum
		float bv = -__builtin_inff();
		int be = 0x7fffffff;
#pragma unroll
		for (int q = 0; q < PER; q++)
			if (v[q] > bv) {
				bv = v[q];
				be = q * 64 + lane;
			}
		// wave argmax by (value desc, index asc)
#pragma unroll
		for (int off = 32; off > 0; off >>= 1) {
			const float ov = __shfl_xor(bv, off);
			const int oe = __shfl_xor(be, off);
			if (ov > bv || (ov == bv && oe < be)) {
				bv = ov;
				be = oe;
			}
		}
		const bool found = bv > -__builtin_inff();
		if (lane == j) {
			my_s = found ? bv : -__builtin_inff();
			my_i = found ? be : -1;
		}
		if (found && (be & 63) == lane) {
#pragma unroll
			for (int q = 0; q < PER; q++)
				if (q == (be >> 6))
					v[q] = -__builtin_inff();
		}
	}
	// softmax over the k selected logits: max is slot 0 (or -inf), exp per lane
	float mx = __shfl(my_s, 0);
	for (int j = 1; j < k; j++) {
		const float sj = __shfl(my_s, j);
		if (sj > mx)
			mx = sj;
	}
	const float ev = lane < k ? tie_expf_tab(my_s - mx, etab) : 0.0f;
	float sum = 0.0f;
	for (int j = 0; j < k; j++)
		sum = sum + __shfl(ev, j);
	const float inv = __fdiv_rn(1.0f, sum);
	if (lane < k) {
		out_w[lane] = ev * inv;
		out_idx[lane] = my_i;
	}
}

// DPP lane moves inside rows of 16 lanes (v_mov_b32 with a DPP control)
template <int CTRL> __device__ __forceinline__ float dppf(float v)
{
	return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL> __device__ __forceinline__ int dppi(int v)
{
	return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
constexpr int DPP_XOR1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <- lane 7-i within each 8
constexpr int DPP_SHL1 = 0x101, DPP_SHL2 = 0x102, DPP_SHL4 = 0x104; // lane i <- lane i+n (row of 16)

// hsum_f32_avx2's tree over the 8 lanes l = lane%8 of a group, on lane l = 0:
// ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7))  (math_avx2.c:14-21)
__device__ __forceinline__ float hsum8_lanes(float v)
{
	const float s = v + dppf<DPP_SHL4>(v); // lanes 0..3: s_m = v_m + v_m+4
	const float a = s + dppf<DPP_SHL1>(s); // lane 0: s0 + s1, lane 2: s2 + s3
	return a + dppf<DPP_SHL2>(a);          // lane 0: (s0 + s1) + (s2 + s3)
}

// The same selection and softmax for 8 tokens per wave: 8 lanes per token
// (E <= 128, 16 logits per lane).  Identical order of selection (value
// descending, index ascending; NaN and -inf never qualify) and identical
// softmax arithmetic: the maximum over the slots, e_j = expf(s_j - max),
// the sum formed serially in slot order, w_j = e_j * (1 / sum).  The
// argmax runs over DPP lane moves.  `lg` is the group's token's E logits,
// `sel` LDS scratch of MAX_K floats for that token.
__device__ __forceinline__ void topk_softmax_group8(const float *lg, int E, int k, float *sel, const uint64_t *etab,
						    int32_t *out_idx, float *out_w)
{
	constexpr int G = 8, V = 16;
	const int lig = threadIdx.x & (G - 1);
	float v[V];
#pragma unroll
	for (int q = 0; q < V; q++) {
		const int e = q * G + lig;
		const float x = e < E ? lg[e] : -__builtin_inff();
		v[q] = (x > -__builtin_inff()) ? x : -__builtin_inff();
	}
	auto better = [](float ov, int oe, float bv, int be) { return ov > bv || (ov == bv && oe < be); };
	for (int j = 0; j < k; j++) {
		float bv = -__builtin_inff();
		int be = 0x7fffffff;
#pragma unroll
		for (int q = 0; q < V; q++)
			if (v[q] > bv) {
				bv = v[q];
				be = q * G + lig;
			}
		float ov = dppf<DPP_XOR1>(bv);
		int oe = dppi<DPP_XOR1>(be);
		if (better(ov, oe, bv, be)) {
			bv = ov;
			be = oe;
		}
		ov = dppf<DPP_XOR2>(bv);
		oe = dppi<DPP_XOR2>(be);
		if (better(ov, oe, bv, be)) {
			bv = ov;
			be = oe;
		}
		ov = dppf<DPP_HALF_MIRROR>(bv);
		oe = dppi<DPP_HALF_MIRROR>(be);
		if (better(ov, oe, bv, be)) {
			bv = ov;
			be = oe;
		}
		const bool found = bv > -__builtin_inff();
		if (lig == 0) {
			sel[j] = found ? bv : -__builtin_inff();
			out_idx[j] = found ? be : -1;
		}
		if (found && (be & (G - 1)) == lig) {
#pragma unroll
			for (int q = 0; q < V; q++)
				if (q == be / G)
					v[q] = -__builtin_inff();
		}
	}
	__builtin_amdgcn_wave_barrier();
	float mx = sel[0];
	for (int j = 1; j < k; j++)
		if (sel[j] > mx)
			mx = sel[j];
	// e_j on lane j % 8, then the serial sum on lane 0
	float ev[MAX_K / G];
#pragma unroll
	for (int q = 0; q < MAX_K / G; q++) {
		const int j = q * G + lig;
		ev[q] = j < k ? tie_expf_tab(sel[j] - mx, etab) : 0.0f;
	}
	__builtin_amdgcn_wave_barrier();
#pragma unroll
	for (int q = 0; q < MAX_K / G; q++) {
		const int j = q * G + lig;
		if (j < k)
			sel[j] = ev[q];
	}
	__builtin_amdgcn_wave_barrier();
	float sum = 0.0f;
	for (int j = 0; j < k; j++)
		sum = sum + sel[j];
	const float inv = __fdiv_rn(1.0f, sum);
#pragma unroll
	for (int q = 0; q < MAX_K / G; q++) {
		const int j = q * G + lig;
		if (j < k)
			out_w[j] = ev[q] * inv;
	}
}

// ------------------------------------------------------------ router_small
constexpr int RS_TOK = 4;     // tokens per workgroup
constexpr int RS_THREADS = 256;

__global__ __launch_bounds__(RS_THREADS) void router_small_kernel(const float *__restrict__ x,
								  const float *__restrict__ W,
								  const float *__restrict__ bias, int T, int d, int E,
								  int k, float *__restrict__ logits,
								  int32_t *__restrict__ topk_idx,
								  float *__restrict__ topk_w, uint32_t *counter)
{
	extern __shared__ float lds[]; // W row [d] | x [RS_TOK][d]
	float *ws = lds;
	float *xs = lds + d;
	__shared__ int s_last;
	__shared__ uint64_t etab[32];

	const int e = blockIdx.x;
	const int t0 = blockIdx.y * RS_TOK;
	const int nt = min(RS_TOK, T - t0);
	const int tid = threadIdx.x;
	const int d4 = d >> 2;

	const float4 *W4 = reinterpret_cast<const float4 *>(W + (size_t)e * d);
	for (int i = tid; i < d4; i += RS_THREADS)
		reinterpret_cast<float4 *>(ws)[i] = W4[i];
	for (int t = 0; t < nt; t++) {
		const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)(t0 + t) * d);
		for (int i = tid; i < d4; i += RS_THREADS)
			reinterpret_cast<float4 *>(xs + (size_t)t * d)[i] = x4[i];
	}
	__syncthreads();

	if (tid < RS_TOK * 8) {
		const int t = tid >> 3, l = tid & 7;
		float acc = 0.0f;
		if (t < nt) {
			const float *xt = xs + (size_t)t * d;
#pragma unroll 8
			for (int i = 0; i < d; i += 8)
				acc = __builtin_fmaf(xt[i + l], ws[i + l], acc);
		}
		// hsum8 across the 8 lanes of this chain group
		float s = acc + __shfl_down(acc, 4, 8);
		float a = s + __shfl_down(s, 1, 8);
		float r = a + __shfl_down(a, 2, 8);
		if (l == 0 && t < nt) {
			if (bias)
				r = r + bias[e];
			logits[(size_t)(t0 + t) * E + e] = r;
		}
	}

	// completion per token group: the last of the E workgroups of this
	// group (counter blockIdx.y, self-resetting) selects the experts of its
	// tokens, one wave per token
	__syncthreads();
	uint32_t *cnt = counter + blockIdx.y;
	if (tid == 0) {
		__threadfence();
		const uint32_t prev = atomicAdd(cnt, 1u);
		s_last = (prev == gridDim.x - 1);
	}
	__syncthreads();
	if (!s_last)
		return;
	if (tid < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		etab[tid] = tab[tid];
	}
	__threadfence();
	__syncthreads();
	const int wave = tid >> 6;
	if (wave < nt) {
		const int t = t0 + wave;
		float *my = lds + (size_t)wave * E;
		for (int q = tid & 63; q < E; q += 64)
			my[q] = __hip_atomic_load(logits + (size_t)t * E + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		__builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
		__builtin_amdgcn_wave_barrier();
		__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
		topk_softmax_wave(my, E, k, etab, topk_idx + (size_t)t * k, topk_w + (size_t)t * k);
	}
	if (tid == 0)
		__hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ router_logits
// One workgroup (8 waves, two per SIMD) per 32 tokens x 32 experts.  Thread
// (l, eg, tg) runs the 16 lane-l chains of experts 4eg..4eg+3 x tokens
// 4tg..4tg+3, each in TIE's order (i ascending): per step one 16-byte LDS
// read of the 4 weights and 4 reads of x feed 16 FMAs.  K advances 256 at
// a time through a double-buffered LDS pipeline filled by direct
// global->LDS loads (global_load_lds_dwordx4): the x rows as they are
// (token-major) and the matching 256 rows x 32 experts of the transposed
// router matrix, whose 16-byte column groups are XOR-swizzled by row
// (conflict-free reads).
constexpr int RT_TOK = 32, RT_EXP = 32, RT_KC = 256, RT_THREADS = 512, RT_NW = RT_THREADS / 64;
constexpr int RT_WBYTES = RT_KC * RT_EXP * 4;   // W^T chunk (32 KiB)
constexpr int RT_XBYTES = RT_TOK * RT_KC * 4;   // x chunk (32 KiB)
constexpr int RT_BUF = RT_WBYTES + RT_XBYTES;
constexpr int RT_LDS = 2 * RT_BUF;              // double-buffered (128 KiB)

__device__ __forceinline__ uint32_t rt_lds_addr(const void *p)
{
	return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
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
		if (t < nt)
			rt_dma16(x + (size_t)(t0 + t) * d + kc + 4 * lane,
				 __builtin_amdgcn_readfirstlane(rt_lds_addr(buf + RT_WBYTES + t * RT_KC * 4)));
	}
}

__device__ __forceinline__ void rt_barrier()
{
	asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__global__ __launch_bounds__(RT_THREADS) void router_logits_kernel(const float *__restrict__ x,
								   const float *__restrict__ WT,
								   const float *__restrict__ bias, int T, int d, int E,
								   float *__restrict__ logits)
{
	extern __shared__ __attribute__((aligned(16))) uint8_t rt_lds[];

	const int tid = threadIdx.x;
	const int l = tid & 7, eg = (tid >> 3) & 7, tg = tid >> 6;
	const int t0 = blockIdx.x * RT_TOK, e0 = blockIdx.y * RT_EXP;
	const int nt = min(RT_TOK, T - t0);
	const int nkc = d / RT_KC;
	// float index of experts 4eg.. in W^T row r: slot eg ^ (r%8), r % 8 == l
	const int wcol = 4 * (eg ^ l);
	const int xo = (4 * tg) * RT_KC + l;

	float acc[4][4];
#pragma unroll
	for (int a = 0; a < 4; a++)
#pragma unroll
		for (int b = 0; b < 4; b++)
			acc[a][b] = 0.0f;

	rt_dma_chunk(x, WT, E, d, t0, e0, nt, 0, rt_lds);
	rt_barrier();
	for (int c = 0; c < nkc; c++) {
		if (c + 1 < nkc)
			rt_dma_chunk(x, WT, E, d, t0, e0, nt, (c + 1) * RT_KC, rt_lds + ((c + 1) & 1) * RT_BUF);
		const float *ws = reinterpret_cast<const float *>(rt_lds + (c & 1) * RT_BUF);
		const float *xs = reinterpret_cast<const float *>(rt_lds + (c & 1) * RT_BUF + RT_WBYTES);
#pragma unroll 8
		for (int i = 0; i < RT_KC / 8; i++) {
			const float4 w4 = *reinterpret_cast<const float4 *>(ws + (8 * i + l) * RT_EXP + wcol);
#pragma unroll
			for (int a = 0; a < 4; a++) {
				const float xv = xs[xo + a * RT_KC + 8 * i];
				acc[a][0] = __builtin_fmaf(xv, w4.x, acc[a][0]);
				acc[a][1] = __builtin_fmaf(xv, w4.y, acc[a][1]);
				acc[a][2] = __builtin_fmaf(xv, w4.z, acc[a][2]);
				acc[a][3] = __builtin_fmaf(xv, w4.w, acc[a][3]);
			}
		}
		rt_barrier();
	}

	// hsum8 over the 8 lanes l of each chain group (math_avx2.c:14-21 order)
#pragma unroll
	for (int a = 0; a < 4; a++) {
#pragma unroll
		for (int b = 0; b < 4; b++) {
			float r = hsum8_lanes(acc[a][b]);
			const int t = 4 * tg + a, e = e0 + 4 * eg + b;
			if (l == 0 && t < nt) {
				if (bias)
					r = r + bias[e];
				logits[(size_t)(t0 + t) * E + e] = r;
			}
		}
	}
}

// ------------------------------------------------------------ router_topk
// 32 tokens per workgroup, 8 lanes per token (E <= 128).
constexpr int RK_TOK = 32, RK_THREADS = 8 * RK_TOK;

__global__ __launch_bounds__(RK_THREADS) void router_topk_kernel(const float *__restrict__ logits, int T, int E,
								 int k, int32_t *__restrict__ topk_idx,
								 float *__restrict__ topk_w)
{
	__shared__ float lg[RK_TOK * 128];
	__shared__ float sel[RK_TOK * MAX_K];
	__shared__ uint64_t etab[32];
	const int tid = threadIdx.x;
	const int t0 = blockIdx.x * RK_TOK;
	const int nt = min(RK_TOK, T - t0);
	if (tid < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		etab[tid] = tab[tid];
	}
	for (int i = tid; i < nt * E; i += RK_THREADS)
		lg[i] = logits[(size_t)t0 * E + i];
	__syncthreads();
	const int t = tid / 8;
	if (t < nt)
		topk_softmax_group8(lg + t * E, E, k, sel + t * MAX_K, etab, topk_idx + (size_t)(t0 + t) * k,
				    topk_w + (size_t)(t0 + t) * k);
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
	hipLaunchKernelGGL(transpose_kernel, dim3((L.d + 31) / 32, (L.E + 31) / 32), dim3(32, 8), 0, s, L.router,
			   (float *)L.routerT, L.E, L.d);
	return hipGetLastError();
}

hipError_t launch_router(const Layer &L, const float *x, int T, int k, float *logits, int32_t *topk_idx,
			 float *topk_w, uint32_t *counter, hipStream_t s)
{
	const int d = L.d, E = L.E;
	// the selection kernel keeps 32 tokens' logits in LDS: E <= 128
	const bool tiled = T > 64 && E % RT_EXP == 0 && E <= 128 && d % RT_KC == 0;
	if (tiled) {
		static bool attr = false;
		if (!attr) {
			const hipError_t err = hipFuncSetAttribute((const void *)router_logits_kernel,
								   hipFuncAttributeMaxDynamicSharedMemorySize, RT_LDS);
			if (err != hipSuccess)
				return err;
			attr = true;
		}
		hipLaunchKernelGGL(router_logits_kernel, dim3((T + RT_TOK - 1) / RT_TOK, E / RT_EXP), dim3(RT_THREADS),
				   RT_LDS, s, x, L.routerT, L.bias, T, d, E, logits);
		hipLaunchKernelGGL(router_topk_kernel, dim3((T + RK_TOK - 1) / RK_TOK), dim3(RK_THREADS), 0, s, logits, T,
				   E, k, topk_idx, topk_w);
		return hipGetLastError();
	}
	const size_t lds = sizeof(float) * (size_t)d * (1 + RS_TOK);
	const size_t lds_need = sizeof(float) * (size_t)(RS_THREADS / 64) * E;
	hipLaunchKernelGGL(router_small_kernel, dim3(E, (T + RS_TOK - 1) / RS_TOK), dim3(RS_THREADS),
			   lds > lds_need ? lds : lds_need, s, x, L.router, L.bias, T, d, E, k, logits, topk_idx,
			   topk_w, counter);
	return hipGetLastError();
}

} // namespace tie
