// dispatch.hip -- token-to-expert grouping and the weighted combine.
//
// Reference: TIE runs the experts of each token as k independent
// process_expert_task jobs (model_qwen3.c:446-456) and never groups tokens
// by expert.  On the GPU the (token, slot) pairs are grouped by expert so
// each expert's weights are streamed from HBM once per call, whatever the
// number of tokens routed to it:
//   counts[e]   pairs routed to expert e
//   offsets[e]  exclusive prefix sum of counts (offsets[E] = valid pairs)
//   pairs[]     pair ids p = t*k + j grouped by expert (order inside an
//               expert is not fixed; every pair is computed independently
//               and written to its own row, so results do not depend on it)
//   active[]    experts with counts > 0 in ascending order; active[E] = n
// The combine then restores token order: out[t] = sum_j g[t][j] * y[t*k+j]
// in slot order j = 0..k-1 with one FMA per term, as model_qwen3.c:459-467
// does (acc starts at +0.0f; slots with no expert contribute nothing).
#include "common.h"

namespace tie {

constexpr int DSP_THREADS = 1024;

// Exclusive prefix sum over the workgroup (DSP_THREADS threads, one value
// each); also returns the total.
__device__ __forceinline__ int block_exclusive_scan(int v, int *wsum, int &total)
{
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	constexpr int NW = DSP_THREADS / 64;
	int x = v;
#pragma unroll
	for (int off = 1; off < 64; off <<= 1) {
		const int y = __shfl_up(x, off);
		if (lane >= off)
			x += y;
	}
	if (lane == 63)
		wsum[wave] = x;
	__syncthreads();
	if (wave == 0) {
		int s = lane < NW ? wsum[lane] : 0;
#pragma unroll
		for (int off = 1; off < NW; off <<= 1) {
			const int y = __shfl_up(s, off);
			if (lane >= off)
				s += y;
		}
		if (lane < NW)
			wsum[lane] = s;
	}
	__syncthreads();
	const int prefix = wave > 0 ? wsum[wave - 1] : 0;
	total = wsum[NW - 1];
	__syncthreads();
	return prefix + x - v;
}

// One workgroup: LDS histogram, parallel scans over the experts, LDS-atomic
// placement of the pairs.  Also writes the MFMA work list (one entry per
// MFMA_MT pairs of each active expert).
__global__ __launch_bounds__(DSP_THREADS) void dispatch_kernel(const int32_t *__restrict__ topk_idx, int npairs,
							       int E, int32_t *__restrict__ counts,
							       int32_t *__restrict__ offsets,
							       int32_t *__restrict__ pairs,
							       int32_t *__restrict__ active,
							       int32_t *__restrict__ tile_e,
							       int32_t *__restrict__ tile_m0,
							       int32_t *__restrict__ ntiles)
{
	extern __shared__ int32_t sm[];
	int32_t *cnt = sm;          // [E]
	int32_t *cur = sm + E;      // [E] running cursor
	__shared__ int wsum[DSP_THREADS / 64];
	const int tid = threadIdx.x;
	for (int e = tid; e < E; e += DSP_THREADS)
		cnt[e] = 0;
	__syncthreads();
	for (int p = tid; p < npairs; p += DSP_THREADS) {
		const int e = topk_idx[p];
		if (e >= 0 && e < E)
			atomicAdd(&cnt[e], 1);
	}
	__syncthreads();
	// E <= MAX_E == DSP_THREADS: one expert per thread
	const int e = tid;
	const int c = e < E ? cnt[e] : 0;
	int total, nact, ntot;
	const int off = block_exclusive_scan(c, wsum, total);
	const int aidx = block_exclusive_scan(c > 0 ? 1 : 0, wsum, nact);
	const int nt = (c + MFMA_MT - 1) / MFMA_MT;
	const int toff = block_exclusive_scan(nt, wsum, ntot);
	if (e < E) {
		offsets[e] = off;
		cur[e] = off;
		counts[e] = c;
		if (c > 0)
			active[aidx] = e;
		// the expert's pairs split evenly over its nt tiles
		const int rpt = nt > 0 ? (c + nt - 1) / nt : 0;
		for (int t = 0; t < nt; t++) {
			tile_e[toff + t] = e;
			tile_m0[toff + t] = t * rpt;
		}
	}
	if (tid == 0) {
		offsets[E] = total;
		active[E] = nact;
		ntiles[0] = ntot;
	}
	__syncthreads();
	for (int p = tid; p < npairs; p += DSP_THREADS) {
		const int ex = topk_idx[p];
		if (ex >= 0 && ex < E)
			pairs[atomicAdd(&cur[ex], 1)] = p;
	}
}

hipError_t launch_dispatch(const Layer &L, int T, int k, const int32_t *topk_idx, Workspace &ws, hipStream_t s)
{
	const size_t lds = sizeof(int32_t) * 2 * (size_t)L.E;
	hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(DSP_THREADS), lds, s, topk_idx, T * k, L.E, ws.counts,
			   ws.offsets, ws.pairs, ws.active, ws.tile_e, ws.tile_m0, ws.ntiles);
	return hipGetLastError();
}

// out[t][c] = fma(g_j, y[t*k+j][c], acc) for j = 0..k-1 (model_qwen3.c:459-467)
__global__ __launch_bounds__(256) void combine_kernel(int T, int d, int k, const float *__restrict__ topk_w,
						      const int32_t *__restrict__ topk_idx,
						      const float *__restrict__ y, float *__restrict__ out)
{
	const int t = blockIdx.y;
	const int c4 = blockIdx.x * blockDim.x + threadIdx.x; // float4 column
	if (c4 * 4 >= d)
		return;
	float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
	for (int j = 0; j < k; j++) {
		if (topk_idx[t * k + j] < 0)
			continue;
		const float g = topk_w[t * k + j];
		const float4 v = reinterpret_cast<const float4 *>(y + ((size_t)t * k + j) * d)[c4];
		acc.x = __builtin_fmaf(g, v.x, acc.x);
		acc.y = __builtin_fmaf(g, v.y, acc.y);
		acc.z = __builtin_fmaf(g, v.z, acc.z);
		acc.w = __builtin_fmaf(g, v.w, acc.w);
	}
	reinterpret_cast<float4 *>(out + (size_t)t * d)[c4] = acc;
}

hipError_t launch_combine(int T, int d, int k, const float *topk_w, const int32_t *topk_idx, const float *y,
			  float *out, hipStream_t s)
{
	if (T == 0)
		return hipSuccess;
	const int n4 = d / 4;
	hipLaunchKernelGGL(combine_kernel, dim3((n4 + 255) / 256, T), dim3(256), 0, s, T, d, k, topk_w, topk_idx, y,
			   out);
	return hipGetLastError();
}

} // namespace tie
