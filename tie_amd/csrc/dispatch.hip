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
#include "route.h"

namespace tie {

constexpr int DSP_THREADS = 1024;

// One workgroup groups all pairs (group_pairs): the exact path's grouping
// for batches too large for route_group_kernel.
constexpr int DSP_STAGE_MAX = 16384; // pairs staged in LDS at most (selections + list: 128 KiB)
__global__ __launch_bounds__(DSP_THREADS) void dispatch_kernel(const int32_t *__restrict__ topk_idx, int npairs,
							       int E, int32_t *__restrict__ offsets,
							       int32_t *__restrict__ pairs,
							       int32_t *__restrict__ active)
{
	extern __shared__ __attribute__((aligned(16))) int32_t sidx[];
	__shared__ __attribute__((aligned(16))) int32_t cnt[MAX_E];
	__shared__ int32_t cur[MAX_E];
	__shared__ int wsum[DSP_THREADS / 64];
	if (npairs > DSP_STAGE_MAX) {
		group_pairs<DSP_THREADS>(topk_idx, npairs, E, cnt, cur, wsum, offsets, pairs, active);
		return;
	}
	// selections in, pair list out, both through LDS: the scattered
	// placement stores hit LDS, and global memory sees only coalesced
	// 16-byte loads and stores
	int32_t *spairs = sidx + ((npairs + 3) & ~3);
	const int n4 = npairs >> 2;
	for (int i = threadIdx.x; i < n4; i += DSP_THREADS)
		reinterpret_cast<int4 *>(sidx)[i] = reinterpret_cast<const int4 *>(topk_idx)[i];
	for (int i = 4 * n4 + threadIdx.x; i < npairs; i += DSP_THREADS)
		sidx[i] = topk_idx[i];
	__syncthreads();
	// pairs[0 .. valid): experts' lists back to back (the invalid selections,
	// if any, were not placed)
	const int valid = group_pairs<DSP_THREADS>(sidx, npairs, E, cnt, cur, wsum, offsets, spairs, active);
	const int v4 = valid >> 2;
	for (int i = threadIdx.x; i < v4; i += DSP_THREADS)
		reinterpret_cast<int4 *>(pairs)[i] = reinterpret_cast<const int4 *>(spairs)[i];
	for (int i = 4 * v4 + threadIdx.x; i < valid; i += DSP_THREADS)
		pairs[i] = spairs[i];
}

hipError_t launch_dispatch(const Layer &L, int T, int k, const int32_t *topk_idx, Workspace &ws, hipStream_t s)
{
	const int npairs = T * k;
	const size_t lds = npairs <= DSP_STAGE_MAX ? sizeof(int32_t) * 2 * (size_t)((npairs + 3) & ~3) : 0;
	static bool attr = false;
	if (!attr) {
		const hipError_t err = hipFuncSetAttribute((const void *)dispatch_kernel,
							   hipFuncAttributeMaxDynamicSharedMemorySize,
							   (int)(sizeof(int32_t) * 2 * DSP_STAGE_MAX));
		if (err != hipSuccess)
			return err;
		attr = true;
	}
	tie_launch(dispatch_kernel, dim3(1), dim3(DSP_THREADS), lds, s, topk_idx, npairs, L.E, ws.offsets,
			   ws.pairs, ws.active);
	return hipGetLastError();
}

// Routing and grouping of a small batch (T*k <= RG_MAX_PAIRS) in one
// workgroup: top-k + softmax of every token from its logits (8 lanes per
// token when E <= 128, else a wave per token), then group_pairs.  Saves
// the separate selection launch.
constexpr int RG_MAX_PAIRS = 4096;
#ifndef TIE_RG_GMAX
#define TIE_RG_GMAX 32
#endif
constexpr int RG_LDS_LOGITS = 8192; // T * E up to this: logits staged in LDS
// G > 0: G lanes per token (E <= 128 and more tokens than waves), else one
// wave per token; separate instances keep each one's registers small
template <int G, bool SIG>
__global__ __launch_bounds__(DSP_THREADS) void route_group_kernel(const float *__restrict__ logits, int T, int E,
								  int k, int32_t *__restrict__ topk_idx,
								  float *__restrict__ topk_w,
								  int32_t *__restrict__ offsets,
								  int32_t *__restrict__ pairs,
								  int32_t *__restrict__ active, int routing,
								  const float *__restrict__ pbias)
{
	__shared__ __attribute__((aligned(16))) int32_t cnt[MAX_E];
	__shared__ int32_t cur[MAX_E];
	__shared__ int wsum[DSP_THREADS / 64];
	__shared__ uint64_t etab[32];
	__shared__ int32_t sidx[RG_MAX_PAIRS];
	__shared__ int lpt[2 * LPT_BINS];
	// the logits of all tokens in LDS (one coalesced copy: a wave that
	// selects for several tokens then waits for global memory once)
	__shared__ __attribute__((aligned(16))) float slg[RG_LDS_LOGITS];
	__shared__ float gsel[(DSP_THREADS / 8) * MAX_K]; // per-token scratch of the 8-lane selection
	const int tid = threadIdx.x;
	if (tid < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		etab[tid] = tab[tid];
	}
	const float *lg = logits;
	if (T * E <= RG_LDS_LOGITS) {
		const int n = T * E;
		for (int i = 4 * tid; i < n; i += 4 * DSP_THREADS) {
			if (i + 4 <= n)
				*reinterpret_cast<float4 *>(slg + i) = *reinterpret_cast<const float4 *>(logits + i);
			else
				for (int j = i; j < n; j++)
					slg[j] = logits[j];
		}
		lg = slg;
	}
	__syncthreads();
	if constexpr (G > 0) {
		for (int t0 = 0; t0 < T; t0 += DSP_THREADS / G) {
			const int t = t0 + tid / G;
			if (t < T)
				topk_softmax_group<SIG, G>(lg + (size_t)t * E, E, k, gsel + (tid / G) * MAX_K, etab,
							   sidx + t * k, topk_w + (size_t)t * k, pbias);
		}
	} else {
		for (int t = tid >> 6; t < T; t += DSP_THREADS / 64)
			topk_softmax(lg + (size_t)t * E, E, k, etab, sidx + t * k, topk_w + (size_t)t * k, routing,
				     pbias);
	}
	__syncthreads();
	const int npairs = T * k;
	for (int p = tid; p < npairs; p += DSP_THREADS)
		topk_idx[p] = sidx[p];
	group_pairs<DSP_THREADS>(sidx, npairs, E, cnt, cur, wsum, offsets, pairs, active, lpt);
}

hipError_t launch_route_group(const Layer &L, int T, int k, const float *logits, Workspace &ws, hipStream_t s)
{
	// lanes per token: the most that still run every token in one pass of
	// the workgroup (more lanes, shorter per-lane chains)
	const bool grp = L.E <= 128 && T > DSP_THREADS / 64, sig = L.routing == ROUTE_SIGMOID;
	int G = TIE_RG_GMAX;
	while (G > 8 && T * G > DSP_THREADS)
		G >>= 1;
	auto kern = route_group_kernel<0, false>;
	if (grp)
		kern = G == 32 ? (sig ? route_group_kernel<32, true> : route_group_kernel<32, false>)
		       : G == 16 ? (sig ? route_group_kernel<16, true> : route_group_kernel<16, false>)
				 : (sig ? route_group_kernel<8, true> : route_group_kernel<8, false>);
	tie_launch(kern, dim3(1), dim3(DSP_THREADS), 0, s, logits, T, L.E, k, ws.topk_idx, ws.topk_w, ws.offsets,
			   ws.pairs, ws.active, L.routing, L.pbias);
	return hipGetLastError();
}

// out[t][c] = fma(g_j, y[t*k+j][c], acc) for j = 0..k-1 (model_qwen3.c:459-467);
// with res: out[t][c] = res[t][c] + acc, the residual add that follows the
// block (dispatch_apply_residual, model_qwen3.c:491, apply_residual_f32_f32_avx2
// math_avx2.c:731-751).  res may be out (the hidden state updated in place).
// Tokens with skip[t] != 0 (skip optional) are left alone: the exact
// recomputation writes their rows afterwards, from res as it was.
__global__ __launch_bounds__(256) void combine_kernel(int T, int d, int k, const float *__restrict__ topk_w,
						      const int32_t *__restrict__ topk_idx,
						      const float *__restrict__ y, const float *res, float *out,
						      const int32_t *__restrict__ skip)
{
	const int t = blockIdx.y;
	if (skip && skip[t])
		return;
	const int c4 = blockIdx.x * blockDim.x + threadIdx.x; // float4 column
	if (c4 * 4 >= d)
		return;
	float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
	constexpr int CG = 8;
	// 8 slots at a time: every row of the group loaded before the first
	// FMA (one memory wait per group, not one per slot), then the FMAs in
	// slot order
	for (int j0 = 0; j0 < k; j0 += CG) {
		float4 v[CG];
		float g[CG];
#pragma unroll
		for (int q = 0; q < CG; q++) {
			const int j = j0 + q;
			const bool on = j < k && topk_idx[t * k + (j < k ? j : 0)] >= 0;
			g[q] = on ? topk_w[t * k + j] : 0.0f;
			// every slot's row is loaded (its address does not wait for
			// topk_idx); a slot without an expert adds nothing
			const size_t row = (size_t)t * k + (j < k ? j : j0);
			v[q] = reinterpret_cast<const float4 *>(y + row * d)[c4];
		}
#pragma unroll
		for (int q = 0; q < CG; q++) {
			const int j = j0 + q;
			if (j < k && topk_idx[t * k + j] >= 0) {
				acc.x = __builtin_fmaf(g[q], v[q].x, acc.x);
				acc.y = __builtin_fmaf(g[q], v[q].y, acc.y);
				acc.z = __builtin_fmaf(g[q], v[q].z, acc.z);
				acc.w = __builtin_fmaf(g[q], v[q].w, acc.w);
			}
		}
	}
	if (res) {
		const float4 h = reinterpret_cast<const float4 *>(res + (size_t)t * d)[c4];
		acc.x = h.x + acc.x;
		acc.y = h.y + acc.y;
		acc.z = h.z + acc.z;
		acc.w = h.w + acc.w;
	}
	reinterpret_cast<float4 *>(out + (size_t)t * d)[c4] = acc;
}

// The same with 8 columns per thread for f16 y scaled by 2^-y_shift (the
// matrix-core path's quantised down; combine8_cols)
__global__ __launch_bounds__(256) void combine16_kernel(int T, int d, int k, const float *__restrict__ topk_w,
							const int32_t *__restrict__ topk_idx, const uint16_t *__restrict__ y,
							float ysc, const float *res, float *out, const int32_t *__restrict__ skip)
{
	const int t = blockIdx.y;
	if (skip && skip[t])
		return;
	const int c8 = blockIdx.x * blockDim.x + threadIdx.x;
	if (c8 * 8 >= d)
		return;
	combine8_cols<true>(t, c8, d, k, topk_w, topk_idx, y, ysc, res, out);
}

hipError_t launch_combine(int T, int d, int k, const float *topk_w, const int32_t *topk_idx, const float *y,
			  float *out, hipStream_t s, const float *res, const int32_t *skip, bool y16, int y_shift)
{
	if (T == 0)
		return hipSuccess;
	if (y16) {
		if (d % 8)
			return hipErrorInvalidValue;
		tie_launch(combine16_kernel, dim3((d / 8 + 255) / 256, T), dim3(256), 0, s, T, d, k, topk_w, topk_idx,
			   reinterpret_cast<const uint16_t *>(y), ldexpf(1.0f, y_shift), res, out, skip);
		return hipGetLastError();
	}
	const int n4 = d / 4;
	tie_launch(combine_kernel, dim3((n4 + 255) / 256, T), dim3(256), 0, s, T, d, k, topk_w, topk_idx, y, res,
			   out, skip);
	return hipGetLastError();
}

} // namespace tie
