// route.h -- expert selection (top-k + softmax) and token-to-expert
// grouping as device routines, shared by the router kernels and the
// small-T expert kernels that route in their prologue.
#pragma once
#include "common.h"
#include "tie_expf.h"

namespace tie {

constexpr int LPT_BINS = 256; // pair-count buckets of the launch order

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
constexpr int DPP_MIRROR = 0x140;      // lane i <- lane 15-i within each 16
constexpr int DPP_SHL1 = 0x101, DPP_SHL2 = 0x102, DPP_SHL4 = 0x104; // lane i <- lane i+n (row of 16)

// hsum_f32_avx2's tree over the 8 lanes l = lane%8 of a group, on lane l = 0:
// ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7))  (math_avx2.c:14-21)
__device__ __forceinline__ float hsum8_lanes(float v)
{
	const float s = v + dppf<DPP_SHL4>(v); // lanes 0..3: s_m = v_m + v_m+4
	const float a = s + dppf<DPP_SHL1>(s); // lane 0: s0 + s1, lane 2: s2 + s3
	return a + dppf<DPP_SHL2>(a);          // lane 0: (s0 + s1) + (s2 + s3)
}

// TIE's router chain for lane l of 8 (mat_vec_row_f32_f32_f32_avx2): acc
// = fma(x[8i + l], w[8i + l], acc) for i ascending.  x and w sit in LDS
// lane-major (stage_lane_major: lane l's elements 8i + l contiguous, rows
// padded to start in different banks), so one 16-byte read brings 4 steps
// and the reads of the next 16 steps are in flight while 16 FMAs run.
__device__ __forceinline__ int lane_major_stride(int d)
{
	return d / 8 + 4;
}
__device__ __host__ __forceinline__ int lane_major_floats(int d)
{
	return 8 * (d / 8 + 4);
}

// x[0..d) (global) -> dst[(f % 8) * stride + f / 8] (LDS), all threads
__device__ __forceinline__ void stage_lane_major(float *dst, const float *src, int d)
{
	const int st = lane_major_stride(d);
	copy_in<4>(reinterpret_cast<const float4 *>(src), d / 4, [&](int q, float4 v) {
		const int f = 4 * q, l = f & 7, i = f >> 3;
		dst[(l + 0) * st + i] = v.x;
		dst[(l + 1) * st + i] = v.y;
		dst[(l + 2) * st + i] = v.z;
		dst[(l + 3) * st + i] = v.w;
	});
}

__device__ __forceinline__ float lane_chain(const float *xs, const float *ws, int d, int l)
{
	typedef float f4 __attribute__((ext_vector_type(4)));
	const int st = lane_major_stride(d), n = d / 8;
	const f4 *xl = reinterpret_cast<const f4 *>(xs + l * st);
	const f4 *wl = reinterpret_cast<const f4 *>(ws + l * st);
	float acc = 0.0f;
	f4 xa[4], wa[4];
#pragma unroll
	for (int u = 0; u < 4; u++) {
		xa[u] = xl[u];
		wa[u] = wl[u];
	}
	for (int i = 0; i < n; i += 16) {
		f4 xb[4], wb[4];
		const int nx = (i + 16 < n ? i + 16 : i) / 4;
#pragma unroll
		for (int u = 0; u < 4; u++) {
			xb[u] = xl[nx + u];
			wb[u] = wl[nx + u];
		}
#pragma unroll
		for (int u = 0; u < 4; u++) {
			acc = __builtin_fmaf(xa[u].x, wa[u].x, acc);
			acc = __builtin_fmaf(xa[u].y, wa[u].y, acc);
			acc = __builtin_fmaf(xa[u].z, wa[u].z, acc);
			acc = __builtin_fmaf(xa[u].w, wa[u].w, acc);
		}
#pragma unroll
		for (int u = 0; u < 4; u++) {
			xa[u] = xb[u];
			wa[u] = wb[u];
		}
	}
	return acc;
}

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b)
{
	return a > b ? a : b;
}
__device__ __forceinline__ uint32_t umin32(uint32_t a, uint32_t b)
{
	return a < b ? a : b;
}

// Wave-wide maximum / minimum, returned in every lane: DPP inside rows of
// 16 lanes (quad swaps, half-row and row mirrors), then v_permlane16_swap
// (rows 0<->1, 2<->3) and v_permlane32_swap (halves).
template <bool MAX> __device__ __forceinline__ uint32_t wave_all(uint32_t m)
{
	auto op = [](uint32_t a, uint32_t b) { return MAX ? umax32(a, b) : umin32(a, b); };
	m = op(m, (uint32_t)dppi<DPP_XOR1>((int)m));
	m = op(m, (uint32_t)dppi<DPP_XOR2>((int)m));
	m = op(m, (uint32_t)dppi<DPP_HALF_MIRROR>((int)m));
	m = op(m, (uint32_t)dppi<DPP_MIRROR>((int)m));
	const auto r16 = __builtin_amdgcn_permlane16_swap(m, m, false, false);
	m = op(r16[0], r16[1]);
	const auto r32 = __builtin_amdgcn_permlane32_swap(m, m, false, false);
	return op(r32[0], r32[1]);
}
__device__ __forceinline__ uint32_t wave_all_umax(uint32_t m)
{
	return wave_all<true>(m);
}
__device__ __forceinline__ uint32_t wave_all_umin(uint32_t m)
{
	return wave_all<false>(m);
}

// Order-preserving integer key of a logit: larger float, larger key.  NaN
// maps to the key of -inf (never selected, like find_top_k's strict
// comparison) and -0 to +0 (they compare equal as floats, so they must tie
// and fall back to the index order).  Every key of a selectable value is
// above KEY_NINF; a removed entry gets key 0.
constexpr uint32_t KEY_NINF = 0x007fffffu;
__device__ __forceinline__ uint32_t logit_key(float x)
{
	if (!(x > -__builtin_inff()))
		return KEY_NINF;
	const uint32_t b = __builtin_bit_cast(uint32_t, x + 0.0f); // -0 -> +0
	return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t k)
{
	return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

constexpr int ROUTE_SOFTMAX = 0, ROUTE_SIGMOID = 1;

// The gate weights of the k selected slots, on lane j of the wave: my_s
// is slot j's logit (softmax) or unbiased p (sigmoid), my_i its expert
// (-inf / -1 on lanes of unfilled slots and lanes >= k).
__device__ __forceinline__ void topk_weights_wave(float my_s, int my_i, int k, const uint64_t *etab, int32_t *out_idx,
						  float *out_w, bool sig)
{
	const int lane = threadIdx.x & 63;
	if (sig) {
		// L1 normalisation of the selected p (unfilled slots add nothing)
		const float pj = my_i >= 0 ? my_s : 0.0f;
		float sum = 0.0f;
		for (int j = 0; j < k; j++)
			sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pj), j));
		const float inv = __fdiv_rn(1.0f, sum + 1e-6f);
		if (lane < k) {
			out_w[lane] = pj * inv;
			out_idx[lane] = my_i;
		}
		return;
	}
	// softmax over the k selected logits: max over the slots, exp per lane
	// (lanes of constant index for k <= 8, the common case)
	auto rl = [](float v, int j) {
		return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), j));
	};
	float mx = rl(my_s, 0);
	if (k <= 8) {
#pragma unroll
		for (int j = 1; j < 8; j++) {
			const float sj = rl(my_s, j);
			if (j < k && sj > mx)
				mx = sj;
		}
	} else {
		for (int j = 1; j < k; j++) {
			const float sj = rl(my_s, j);
			if (sj > mx)
				mx = sj;
		}
	}
	const float ev = lane < k ? tie_expf_tab(my_s - mx, etab) : 0.0f;
	float sum = 0.0f;
	if (k <= 8) {
#pragma unroll
		for (int j = 0; j < 8; j++)
			if (j < k)
				sum = sum + rl(ev, j);
	} else {
		for (int j = 0; j < k; j++)
			sum = sum + rl(ev, j);
	}
	const float inv = __fdiv_rn(1.0f, sum);
	if (lane < k) {
		out_w[lane] = ev * inv;
		out_idx[lane] = my_i;
	}
}

// Expert selection of one token, by one wave; PER logits per lane (E <= 64
// * PER), entry e = 64q + lane in register q.
//
// ROUTE_SOFTMAX (Qwen3, model_qwen3.c:431-443): top-k over the logits
// (find_top_k, engine.c:891-914), then softmax over the k selected
// (engine.c:864-888): the maximum over the slots, e_j = expf(s_j - max) on
// lane j, the sum formed serially in slot order, w_j = e_j * (1 / sum).
//
// ROUTE_SIGMOID (LFM2, model_lfm2.c:437-467): p_e = 1 / (1 + expf(-l_e));
// top-k over p_e + bias_e (bias optional, selection only); the weights are
// the unbiased p of the selected experts, L1-normalised: the sum formed
// serially in slot order, w_j = p_j * (1 / (sum + 1e-6)).
//
// The k winners are extracted one at a time under the order (value
// descending, index ascending) -- the order find_top_k's strict-greater
// insertion produces -- by wave-wide maximum of the keys and minimum of
// the indices holding it, both kept in the vector unit (DPP inside rows,
// then gfx950's row-pair and half swaps), so a round has no vector-to-
// scalar round trip.  NaN and -inf never qualify; unfilled slots are
// {-1, -inf} with weight 0.  `lg` and `pbias` may be
// global or LDS memory.
template <int PER>
__device__ __forceinline__ void topk_softmax_wave(const float *lg, int E, int k, const uint64_t *etab,
						  int32_t *out_idx, float *out_w, int routing = ROUTE_SOFTMAX,
						  const float *pbias = nullptr)
{
	const int lane = threadIdx.x & 63;
	const bool sig = routing == ROUTE_SIGMOID;
	uint32_t key[PER];
	float prob[PER]; // sigmoid routing: the unbiased p of each entry
#pragma unroll
	for (int q = 0; q < PER; q++) {
		const int e = q * 64 + lane;
		float v = e < E ? lg[e] : -__builtin_inff();
		prob[q] = 0.0f;
		if (sig && e < E) {
			prob[q] = __fdiv_rn(1.0f, 1.0f + tie_expf_tab(-v, etab));
			v = pbias ? prob[q] + pbias[e] : prob[q];
		}
		key[q] = logit_key(v);
	}
	float my_s = -__builtin_inff();
	int my_i = -1;
	for (int j = 0; j < k; j++) {
		// wave maximum of the keys, in every lane: lane-local, then DPP
		// inside rows of 16, then the row-pair and half swaps
		uint32_t m = key[0];
#pragma unroll
		for (int q = 1; q < PER; q++)
			m = umax32(m, key[q]);
		const uint32_t best = wave_all_umax(m);
		// lowest index holding it (the lowest register first: register q
		// holds indices 64q + lane)
		uint32_t ci = 0xffffffffu;
#pragma unroll
		for (int q = PER - 1; q >= 0; q--)
			if (key[q] == best)
				ci = 64 * q + lane;
		const uint32_t be = wave_all_umin(ci);
		const bool found = best > KEY_NINF; // wave-uniform
		float sv = key_logit(best);
		if (sig) {
			// the winner's unbiased p, from its lane: every lane holds its
			// own candidate's p, the winner's reaches all lanes by the
			// same minimum (only the winner offers a finite index)
			float pv = 0.0f;
#pragma unroll
			for (int q = 0; q < PER; q++)
				if ((uint32_t)(64 * q + lane) == be)
					pv = prob[q];
			sv = __builtin_bit_cast(float, wave_all_umax(ci == be ? __builtin_bit_cast(uint32_t, pv) : 0u));
		}
		if (found && lane == j) {
			my_s = sv;
			my_i = (int)be;
		}
#pragma unroll
		for (int q = 0; q < PER; q++)
			if ((uint32_t)(64 * q + lane) == be)
				key[q] = 0;
	}
	topk_weights_wave(my_s, my_i, k, etab, out_idx, out_w, sig);
}

// The same selection by a whole workgroup, by ranks instead of k rounds of
// wave-wide maxima: entry e's rank is the number of entries before it in
// the order (value descending, index ascending), i.e. with a larger
// composite key {logit_key, ~e}; the entries of rank < k that qualify
// (key above KEY_NINF) take slot = rank.  The E x E comparisons are spread
// over the whole workgroup (P = blockDim / E threads per entry, each
// counting a contiguous 1/P of the entries).  Then wave 0 forms the
// weights (topk_weights_wave).  Usage, E <= RANK_MAX_E <= blockDim:
//   rank_key(v, e, ...) by thread e < E with its logit v, then
//   topk_rank_block(...) (which begins and ends with a barrier).
constexpr int RANK_MAX_E = 128;
struct RankScratch {
	alignas(16) unsigned long long ck[RANK_MAX_E];
	float prob[RANK_MAX_E];
	int cnt[4][RANK_MAX_E];
	float sv[MAX_K];
	int si[MAX_K];
};
__device__ __forceinline__ void rank_key(float v, int e, int routing, const float *pbias, const uint64_t *etab,
					 RankScratch &S)
{
	float p = 0.0f;
	if (routing == ROUTE_SIGMOID) {
		p = __fdiv_rn(1.0f, 1.0f + tie_expf_tab(-v, etab));
		v = pbias ? p + pbias[e] : p;
	}
	S.ck[e] = ((unsigned long long)logit_key(v) << 32) | (uint32_t)~(uint32_t)e;
	S.prob[e] = p;
}
// The gate weights of a selection made by topk_rank_block(..., false)
// (whose slot values S.sv / S.si it reads): out_idx / out_w as
// topk_rank_block(..., true) writes them.  Ends with a barrier.
__device__ __forceinline__ void topk_rank_weights(int k, const uint64_t *etab, int32_t *out_idx, float *out_w,
						  int routing, const RankScratch &S)
{
	const int tid = threadIdx.x;
	if (tid < 64) {
		const float my_s = tid < k ? S.sv[tid] : -__builtin_inff();
		const int my_i = tid < k ? S.si[tid] : -1;
		topk_weights_wave(my_s, my_i, k, etab, out_idx, out_w, routing == ROUTE_SIGMOID);
	}
	__syncthreads();
}

__device__ __forceinline__ void topk_rank_block(int E, int k, const uint64_t *etab, int32_t *out_idx, float *out_w,
						int routing, RankScratch &S, bool weights = true)
{
	const int tid = threadIdx.x;
	const bool sig = routing == ROUTE_SIGMOID;
	if (tid < k) {
		S.sv[tid] = -__builtin_inff();
		S.si[tid] = -1;
	}
	__syncthreads();
	int P = (int)blockDim.x / E;
	P = P > 4 ? 4 : P;
	if (E == RANK_MAX_E && P >= 2) {
		// 2 x 64 comparisons per entry, wave-uniform halves (E = 128 is
		// two waves), fully unrolled 16-byte broadcast reads
		P = 2;
		if (tid < 2 * E) {
			const int p = tid / E, i = tid - p * E;
			const unsigned long long c = S.ck[i];
			const ulonglong2 *q = reinterpret_cast<const ulonglong2 *>(S.ck) + 32 * p;
			int n = 0;
#pragma unroll
			for (int j = 0; j < 32; j++) {
				const ulonglong2 v = q[j];
				n += (v.x > c ? 1 : 0) + (v.y > c ? 1 : 0);
			}
			S.cnt[p][i] = n;
		}
	} else if (tid < P * E) {
		const int p = tid / E, i = tid - p * E;
		const int lo = p * E / P, hi = (p + 1) * E / P;
		const unsigned long long c = S.ck[i];
		int n = 0;
#pragma unroll 8
		for (int j = lo; j < hi; j++)
			n += S.ck[j] > c ? 1 : 0;
		S.cnt[p][i] = n;
	}
	__syncthreads();
	if (tid < E) {
		int n = 0;
		for (int p = 0; p < P; p++)
			n += S.cnt[p][tid];
		const uint32_t key = (uint32_t)(S.ck[tid] >> 32);
		if (n < k && key > KEY_NINF) {
			S.sv[n] = sig ? S.prob[tid] : key_logit(key);
			S.si[n] = tid;
		}
	}
	__syncthreads();
	if (!weights) {
		// the experts only (the weights later, by topk_rank_weights)
		if (tid < k)
			out_idx[tid] = S.si[tid];
		__syncthreads();
		return;
	}
	topk_rank_weights(k, etab, out_idx, out_w, routing, S);
}

// topk_softmax_wave with PER chosen for E (E <= MAX_E)
__device__ __forceinline__ void topk_softmax(const float *lg, int E, int k, const uint64_t *etab, int32_t *out_idx,
					     float *out_w, int routing, const float *pbias)
{
	if (E <= 64)
		topk_softmax_wave<1>(lg, E, k, etab, out_idx, out_w, routing, pbias);
	else if (E <= 128)
		topk_softmax_wave<2>(lg, E, k, etab, out_idx, out_w, routing, pbias);
	else if (E <= 256)
		topk_softmax_wave<4>(lg, E, k, etab, out_idx, out_w, routing, pbias);
	else if (E <= 512)
		topk_softmax_wave<8>(lg, E, k, etab, out_idx, out_w, routing, pbias);
	else
		topk_softmax_wave<16>(lg, E, k, etab, out_idx, out_w, routing, pbias);
}

// The same selection for 64 / G tokens per wave: G lanes per token (G in
// {8, 16, 32}; E <= 128, 128 / G entries per lane, entry e = G q + lane % G
// in register q), so a wave runs the rounds of several tokens at once (a
// round is a chain of dependent vector operations; one token per wave
// leaves the SIMD mostly idle).  Identical order of selection (the same
// keys: value descending, index ascending; NaN and -inf never qualify) and
// identical weight arithmetic for both routings.  The argmax of a round runs
// over lane moves inside the G lanes.  `sel`: LDS scratch of MAX_K floats
// for the token.
template <bool SIG, int G>
__device__ __forceinline__ void topk_softmax_group(const float *lg, int E, int k, float *sel, const uint64_t *etab,
						   int32_t *out_idx, float *out_w, const float *pbias)
{
	static_assert(G == 8 || G == 16 || G == 32, "8, 16 or 32 lanes per token");
	constexpr int V = 128 / G;
	const int lig = threadIdx.x & (G - 1);
	constexpr bool sig = SIG;
	uint32_t key[V];
	float prob[V];
#pragma unroll
	for (int q = 0; q < V; q++) {
		const int e = q * G + lig;
		float v = e < E ? lg[e] : -__builtin_inff();
		prob[q] = 0.0f;
		if constexpr (SIG) {
			if (e < E) {
				prob[q] = __fdiv_rn(1.0f, 1.0f + tie_expf_tab(-v, etab));
				v = pbias ? prob[q] + pbias[e] : prob[q];
			}
		}
		key[q] = logit_key(v);
	}
	auto better = [](uint32_t ok, int oe, uint32_t bk, int be) { return ok > bk || (ok == bk && oe < be); };
	for (int j = 0; j < k; j++) {
		// the lane's best (largest key, lowest index on ties) as a tree over
		// adjacent ranges (the left range always holds the lower indices, so
		// the right one wins only when strictly larger): depth 4, not 16
		uint32_t tk[V];
		int tq[V];
#pragma unroll
		for (int q = 0; q < V; q++) {
			tk[q] = key[q];
			tq[q] = q;
		}
#pragma unroll
		for (int w = 1; w < V; w <<= 1)
#pragma unroll
			for (int q = 0; q < V; q += 2 * w)
				if (tk[q + w] > tk[q]) {
					tk[q] = tk[q + w];
					tq[q] = tq[q + w];
				}
		uint32_t bk = tk[0];
		int be = bk > 0 ? tq[0] * G + lig : 0x7fffffff;
		uint32_t ok = (uint32_t)dppi<DPP_XOR1>((int)bk);
		int oe = dppi<DPP_XOR1>(be);
		if (better(ok, oe, bk, be)) {
			bk = ok;
			be = oe;
		}
		ok = (uint32_t)dppi<DPP_XOR2>((int)bk);
		oe = dppi<DPP_XOR2>(be);
		if (better(ok, oe, bk, be)) {
			bk = ok;
			be = oe;
		}
		ok = (uint32_t)dppi<DPP_HALF_MIRROR>((int)bk);
		oe = dppi<DPP_HALF_MIRROR>(be);
		if (better(ok, oe, bk, be)) {
			bk = ok;
			be = oe;
		}
		if constexpr (G >= 16) {
			ok = (uint32_t)dppi<DPP_MIRROR>((int)bk);
			oe = dppi<DPP_MIRROR>(be);
			if (better(ok, oe, bk, be)) {
				bk = ok;
				be = oe;
			}
		}
		if constexpr (G >= 32) {
			ok = (uint32_t)__shfl_xor((int)bk, 16);
			oe = __shfl_xor(be, 16);
			if (better(ok, oe, bk, be)) {
				bk = ok;
				be = oe;
			}
		}
		const bool found = bk > KEY_NINF;
		if (found && (be & (G - 1)) == lig) {
			// the winner's lane records the slot and removes the entry
			float pv = 0.0f;
#pragma unroll
			for (int q = 0; q < V; q++)
				if (q == be / G) {
					pv = prob[q];
					key[q] = 0;
				}
			sel[j] = sig ? pv : key_logit(bk);
			out_idx[j] = be;
		} else if (!found && lig == 0) {
			sel[j] = -__builtin_inff();
			out_idx[j] = -1;
		}
	}
	__builtin_amdgcn_wave_barrier();
	if constexpr (SIG) {
		// L1 normalisation of the selected p (unfilled slots add nothing)
		float sum = 0.0f;
		for (int j = 0; j < k; j++)
			sum = sum + (sel[j] > -__builtin_inff() ? sel[j] : 0.0f);
		const float inv = __fdiv_rn(1.0f, sum + 1e-6f);
		for (int j = lig; j < k; j += G)
			out_w[j] = (sel[j] > -__builtin_inff() ? sel[j] : 0.0f) * inv;
		return;
	}
	float mx = sel[0];
	for (int j = 1; j < k; j++)
		if (sel[j] > mx)
			mx = sel[j];
	// e_j on lane j % G, then the serial sum
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

// Exclusive prefix sum over a workgroup of NT threads (one value each);
// `total` receives the sum.  wsum: LDS scratch of NT/64 ints.
// The same over 64-bit values (two counts packed in one word: neither
// half carries into the other while both stay non-negative and below 2^31
// in total).
template <int NT>
__device__ __forceinline__ long long block_exclusive_scan64(long long v, long long *wsum, long long &total)
{
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	constexpr int NW = NT / 64;
	long long x = v;
#pragma unroll
	for (int off = 1; off < 64; off <<= 1) {
		const long long y = __shfl_up(x, off);
		if (lane >= off)
			x += y;
	}
	if (lane == 63)
		wsum[wave] = x;
	__syncthreads();
	long long prefix = 0;
#pragma unroll
	for (int i = 0; i < NW; i++)
		prefix += i < wave ? wsum[i] : 0;
	total = 0;
#pragma unroll
	for (int i = 0; i < NW; i++)
		total += wsum[i];
	__syncthreads();
	return prefix + x - v;
}

template <int NT> __device__ __forceinline__ int block_exclusive_scan(int v, int *wsum, int &total)
{
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	constexpr int NW = NT / 64;
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

// Groups the pairs p = t*k + j by expert, by one workgroup of NT >= E
// threads, and returns the number of valid pairs.  `idx` holds the
// selected expert of every pair (-1: none).  Writes offsets[0..E]
// (exclusive prefix sum of the per-expert counts; offsets[E] = valid
// pairs), pairs[] (pair ids grouped by expert; the order inside an expert
// is not fixed: every pair is computed on its own row, so results do not
// depend on it) and active[0..E] (experts with pairs, by descending pair
// count with lpt -- ties in any order --, else ascending; active[E] =
// their number).  cnt / cur: LDS scratch of E ints each; wsum:
// LDS scratch of NT/64 ints.  Output pointers may be LDS or global memory.
template <int NT>
__device__ __forceinline__ int group_pairs(const int32_t *idx, int npairs, int E, int32_t *cnt, int32_t *cur,
					    int *wsum, int32_t *offsets, int32_t *pairs, int32_t *active,
					    int *lpt = nullptr)
{
	const int tid = threadIdx.x;
	for (int e = tid; e < E; e += NT)
		cnt[e] = 0;
	__syncthreads();
	for (int p = tid; p < npairs; p += NT) {
		const int e = idx[p];
		if (e >= 0 && e < E)
			atomicAdd(&cnt[e], 1);
	}
	__syncthreads();
	if (E <= 128 && npairs < 32768) {
		// one wave: experts 2 lane, 2 lane + 1; counts and active flags
		// scanned together (counts in the high half), then the LPT slots
		if (tid < 64) {
			const int e0 = 2 * tid, e1 = e0 + 1;
			const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
			const int v = ((c0 + c1) << 16) | ((c0 > 0) + (c1 > 0));
			int inc = v;
#pragma unroll
			for (int o = 1; o < 64; o <<= 1) {
				const int y = __shfl_up(inc, o);
				if (tid >= o)
					inc += y;
			}
			const int ex = inc - v, all = __shfl(inc, 63);
			const int off0 = ex >> 16, off1 = off0 + c0;
			int r0 = ex & 0xffff, r1 = r0 + (c0 > 0);
			if (lpt) {
				// rank by pair count, larger first: counts bucketed (the last
				// bucket shared), slots inside a bucket by LDS atomics
				int *hist = lpt, *bcur = lpt + LPT_BINS;
				for (int i = tid; i < LPT_BINS; i += 64)
					hist[i] = 0;
				__builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
				__builtin_amdgcn_wave_barrier();
				const int b0 = LPT_BINS - 1 - (c0 < LPT_BINS - 1 ? c0 : LPT_BINS - 1);
				const int b1 = LPT_BINS - 1 - (c1 < LPT_BINS - 1 ? c1 : LPT_BINS - 1);
				if (c0 > 0)
					atomicAdd(&hist[b0], 1);
				if (c1 > 0)
					atomicAdd(&hist[b1], 1);
				__builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
				__builtin_amdgcn_wave_barrier();
				// exclusive scan of the buckets, LPT_BINS / 64 per lane
				constexpr int BPL = LPT_BINS / 64;
				int h[BPL], hs = 0;
#pragma unroll
				for (int i = 0; i < BPL; i++) {
					h[i] = hist[BPL * tid + i];
					hs += h[i];
				}
				int hin = hs;
#pragma unroll
				for (int o = 1; o < 64; o <<= 1) {
					const int y = __shfl_up(hin, o);
					if (tid >= o)
						hin += y;
				}
				int base = hin - hs;
#pragma unroll
				for (int i = 0; i < BPL; i++) {
					bcur[BPL * tid + i] = base;
					base += h[i];
				}
				__builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
				__builtin_amdgcn_wave_barrier();
				if (c0 > 0)
					r0 = atomicAdd(&bcur[b0], 1);
				if (c1 > 0)
					r1 = atomicAdd(&bcur[b1], 1);
			}
			if (e0 < E) {
				offsets[e0] = off0;
				cur[e0] = off0;
				if (c0 > 0)
					active[r0] = e0;
			}
			if (e1 < E) {
				offsets[e1] = off1;
				cur[e1] = off1;
				if (c1 > 0)
					active[r1] = e1;
			}
			if (tid == 0) {
				offsets[E] = all >> 16;
				active[E] = all & 0xffff;
				wsum[0] = all >> 16;
			}
		}
		__syncthreads();
		const int total = wsum[0];
		for (int p = tid; p < npairs; p += NT) {
			const int ex = idx[p];
			if (ex >= 0 && ex < E)
				pairs[atomicAdd(&cur[ex], 1)] = p;
		}
		__syncthreads();
		return total;
	}
	const int e = tid;
	const int c = e < E ? cnt[e] : 0;
	int total, nact;
	const int off = block_exclusive_scan<NT>(c, wsum, total);
	const int aidx = block_exclusive_scan<NT>(c > 0 ? 1 : 0, wsum, nact);
	// lpt (LDS scratch of 2 * LPT_BINS ints, or null): active experts
	// ordered by pair count, largest first, ties in no fixed order (so only
	// for a grouping made once and shared by all readers): the expert
	// kernels launch one workgroup per active slot in this order, so the
	// longest workgroups start first.  Otherwise ascending expert index.
	int rank = aidx;
	if (lpt) {
		// bucket the experts by pair count (larger counts first; counts past
		// the last bucket share it), then take slots inside a bucket by an
		// LDS atomic: that order only decides which workgroup launches
		// first, never a result
		constexpr int NBIN = NT < LPT_BINS ? NT : LPT_BINS;
		int *lpt_hist = lpt, *lpt_cur = lpt + NBIN;
		for (int i = tid; i < NBIN; i += NT)
			lpt_hist[i] = 0;
		__syncthreads();
		const int bin = NBIN - 1 - (c < NBIN - 1 ? c : NBIN - 1);
		if (e < E && c > 0)
			atomicAdd(&lpt_hist[bin], 1);
		__syncthreads();
		int nb_tot;
		const int base = block_exclusive_scan<NT>(tid < NBIN ? lpt_hist[tid] : 0, wsum, nb_tot);
		if (tid < NBIN)
			lpt_cur[tid] = base;
		__syncthreads();
		if (e < E && c > 0)
			rank = atomicAdd(&lpt_cur[bin], 1);
	}
	if (e < E) {
		offsets[e] = off;
		cur[e] = off;
		if (c > 0)
			active[rank] = e;
	}
	if (tid == 0) {
		offsets[E] = total;
		active[E] = nact;
	}
	__syncthreads();
	for (int p = tid; p < npairs; p += NT) {
		const int ex = idx[p];
		if (ex >= 0 && ex < E)
			pairs[atomicAdd(&cur[ex], 1)] = p;
	}
	__syncthreads();
	return total;
}

} // namespace tie
