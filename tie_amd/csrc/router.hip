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
// Two shapes of the logit computation:
//   router_small  one workgroup per (expert, group of 4 tokens); the expert
//                 row and the tokens are staged in LDS with coalesced
//                 16-byte loads, one thread per (token, lane) runs the
//                 256-long FMA chain.  Used for small T, where spreading the
//                 1 MiB router matrix over E workgroups matters most.  The
//                 last workgroup to finish (grid-completion counter,
//                 self-resetting) does top-k + softmax for every token.
//   router_tiled  one workgroup per 8 tokens and all experts; K is walked
//                 in 64-wide chunks staged in LDS; each thread owns two of
//                 an expert's 8 lane chains for the 8 tokens.  Top-k and
//                 softmax run in the same workgroup, one wave per token.
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
__device__ void topk_softmax_wave(const float *lg, int E, int k, int32_t *out_idx, float *out_w)
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
	const float ev = lane < k ? tie_expf(my_s - mx) : 0.0f;
	float sum = 0.0f;
	for (int j = 0; j < k; j++)
		sum = sum + __shfl(ev, j);
	const float inv = __fdiv_rn(1.0f, sum);
	if (lane < k) {
		out_w[lane] = ev * inv;
		out_idx[lane] = my_i;
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
	__threadfence();
	const int wave = tid >> 6;
	if (wave < nt) {
		const int t = t0 + wave;
		float *my = lds + (size_t)wave * E;
		for (int q = tid & 63; q < E; q += 64)
			my[q] = __hip_atomic_load(logits + (size_t)t * E + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		__builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
		__builtin_amdgcn_wave_barrier();
		__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
		topk_softmax_wave(my, E, k, topk_idx + (size_t)t * k, topk_w + (size_t)t * k);
	}
	if (tid == 0)
		__hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ router_tiled
constexpr int RT_TOK = 8;   // tokens per workgroup
constexpr int RT_KC = 64;   // K chunk
constexpr int RT_WPAD = 4;  // LDS row padding (floats) against bank conflicts

__global__ __launch_bounds__(1024) void router_tiled_kernel(const float *__restrict__ x, const float *__restrict__ W,
							    const float *__restrict__ bias, int T, int d, int E,
							    int k, int32_t *__restrict__ topk_idx,
							    float *__restrict__ topk_w, float *__restrict__ logits_out)
{
	extern __shared__ float lds[];
	const int wst = RT_KC + RT_WPAD;
	float *wsm = lds;                      // [E][wst]
	float *xsm = wsm + (size_t)E * wst;    // [RT_TOK][RT_KC]
	float *lgm = xsm + RT_TOK * RT_KC;     // [RT_TOK][E]

	const int tid = threadIdx.x;
	const int nthr = blockDim.x; // 4 * E
	const int e = tid >> 2, q = tid & 3; // chains 2q, 2q+1
	const int t0 = blockIdx.x * RT_TOK;
	const int nt = min(RT_TOK, T - t0);

	float acc[RT_TOK][2];
#pragma unroll
	for (int t = 0; t < RT_TOK; t++)
		acc[t][0] = acc[t][1] = 0.0f;

	for (int kc = 0; kc < d; kc += RT_KC) {
		__syncthreads();
		// stage W[:, kc:kc+64] and x[t0:t0+8, kc:kc+64]
		for (int i = tid; i < E * (RT_KC / 4); i += nthr) {
			const int r = i / (RT_KC / 4), c = i % (RT_KC / 4);
			const float4 v = *reinterpret_cast<const float4 *>(W + (size_t)r * d + kc + 4 * c);
			*reinterpret_cast<float4 *>(wsm + (size_t)r * wst + 4 * c) = v;
		}
		for (int i = tid; i < RT_TOK * (RT_KC / 4); i += nthr) {
			const int t = i / (RT_KC / 4), c = i % (RT_KC / 4);
			float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
			if (t < nt)
				v = *reinterpret_cast<const float4 *>(x + (size_t)(t0 + t) * d + kc + 4 * c);
			*reinterpret_cast<float4 *>(xsm + t * RT_KC + 4 * c) = v;
		}
		__syncthreads();
#pragma unroll
		for (int i = 0; i < RT_KC; i += 8) {
			const float2 w2 = *reinterpret_cast<const float2 *>(wsm + (size_t)e * wst + i + 2 * q);
#pragma unroll
			for (int t = 0; t < RT_TOK; t++) {
				const float2 x2 = *reinterpret_cast<const float2 *>(xsm + t * RT_KC + i + 2 * q);
				acc[t][0] = __builtin_fmaf(x2.x, w2.x, acc[t][0]);
				acc[t][1] = __builtin_fmaf(x2.y, w2.y, acc[t][1]);
			}
		}
	}

	// hsum8: lanes l = 2q + c.  s_m = v[m] + v[m+4]: thread q in {0,1} takes
	// v[2q+c] + v[2q+4+c] from thread q+2; a = s0 + s1 on q=0, b = s2 + s3
	// on q=1; r = a + b on q=0.
#pragma unroll
	for (int t = 0; t < RT_TOK; t++) {
		const float o0 = __shfl_down(acc[t][0], 2, 4);
		const float o1 = __shfl_down(acc[t][1], 2, 4);
		const float s0 = acc[t][0] + o0; // q=0: s0, q=1: s2
		const float s1 = acc[t][1] + o1; // q=0: s1, q=1: s3
		const float ab = s0 + s1;        // q=0: a,  q=1: b
		const float b = __shfl_down(ab, 1, 4);
		float r = ab + b;
		if (q == 0 && t < nt) {
			if (bias)
				r = r + bias[e];
			lgm[t * E + e] = r;
			if (logits_out)
				logits_out[(size_t)(t0 + t) * E + e] = r;
		}
	}
	__syncthreads();
	const int wave = tid >> 6;
	const int nw = nthr >> 6;
	for (int t = wave; t < nt; t += nw) {
		topk_softmax_wave(lgm + t * E, E, k,
				  topk_idx + (size_t)(t0 + t) * k, topk_w + (size_t)(t0 + t) * k);
		__builtin_amdgcn_wave_barrier();
	}
}

hipError_t launch_router(const Layer &L, const float *x, int T, int k, float *logits, int32_t *topk_idx,
			 float *topk_w, uint32_t *counter, hipStream_t s)
{
	const int d = L.d, E = L.E;
	const bool tiled = (T > 64) && (E % 16 == 0) && (4 * E <= 1024) && (E >= 16);
	if (tiled) {
		const int nthr = 4 * E;
		const size_t lds = sizeof(float) * ((size_t)E * (RT_KC + RT_WPAD) + RT_TOK * RT_KC + RT_TOK * E) +
				   sizeof(int) * 16 * MAX_K + sizeof(float) * 16 * MAX_K;
		hipLaunchKernelGGL(router_tiled_kernel, dim3((T + RT_TOK - 1) / RT_TOK), dim3(nthr), lds, s, x, L.router,
				   L.bias, T, d, E, k, topk_idx, topk_w, logits);
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
