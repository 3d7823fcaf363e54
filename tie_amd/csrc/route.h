// route.h -- expert selection (top-k + softmax) and token-to-expert
// grouping as device routines, shared by the router kernels and the
// small-T expert kernels that route in their prologue.
#pragma once
#include "common.h"
#include "tie_expf.h"

namespace tie {

constexpr int LPT_BINS = 256; // pair-count buckets of the launch order

// top-k (engine.c:891-914 semantics) + softmax (engine.c:864-888) for one
// token, by one wave.  `lg` holds the token's E logits.  The k winners are
// extracted one at a time by a wave-wide argmax under the order (value
// descending, index ascending) -- the order find_top_k's strict-greater
// insertion produces; NaN and -inf never qualify; unfilled slots are
// {-1, -inf}.  Slot j's exponential is computed by lane j, the sum is
// formed serially in slot order, and every weight is e_j * (1 / sum).
__device__ __forceinline__ void topk_softmax_wave(const float *lg, int E, int k, const uint64_t *etab, int32_t *out_idx,
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

// Exclusive prefix sum over a workgroup of NT threads (one value each);
// `total` receives the sum.  wsum: LDS scratch of NT/64 ints.
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
// their number).  With tile_e non-null it also writes the two MFMA work
// lists (list l at offset l * tile_cap): each active expert's pairs split
// evenly over ceil(count / MT) tiles, MT = MFMA_MT_GU (list 0, gate/up) or
// MFMA_MT_DN (list 1, down).  cnt / cur: LDS scratch of E ints each; wsum:
// LDS scratch of NT/64 ints.  Output pointers may be LDS or global memory.
template <int NT>
__device__ __forceinline__ int group_pairs(const int32_t *idx, int npairs, int E, int32_t *cnt, int32_t *cur,
					    int *wsum, int32_t *offsets, int32_t *pairs, int32_t *active,
					    int32_t *tile_e, int32_t *tile_m0, int32_t *ntiles, int *lpt = nullptr,
					    int tile_cap = 0)
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
	if (tile_e) {
		// two lists (gate/up tiles of MFMA_MT_GU rows, down tiles of
		// MFMA_MT_DN rows), list l at tile_e + l * tile_cap
#pragma unroll
		for (int l = 0; l < 2; l++) {
			const int mt = l == 0 ? MFMA_MT_GU : MFMA_MT_DN;
			int ntot;
			const int nt = (c + mt - 1) / mt;
			const int toff = block_exclusive_scan<NT>(nt, wsum, ntot);
			if (e < E) {
				const int rpt = nt > 0 ? (c + nt - 1) / nt : 0;
				for (int t = 0; t < nt; t++) {
					tile_e[l * tile_cap + toff + t] = e;
					tile_m0[l * tile_cap + toff + t] = t * rpt;
				}
			}
			if (tid == 0)
				ntiles[l] = ntot;
		}
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
