// mfma.hip -- grouped expert GEMMs on the bf16 matrix cores (large T).
//
// Reference: TIE runs every (token, expert) pair as three GEMVs
// (process_expert_task, engine.c:916-964) with no reuse of an expert's
// weights across tokens.  For large T the pairs are grouped by expert
// (dispatch.hip) and each expert's weights are dequantised once and
// multiplied against all of its tokens with v_mfma_f32_32x32x16_bf16:
//
//   gate/up:  G = X_e Wg_e^T, U = X_e Wu_e^T, h = silu_tab(G) * U  (fused)
//   down:     Y = h_e Wd_e^T, scattered to the pairs' rows of y
//
// Tiles: a workgroup (8 waves) owns up to MT = 256 pair rows of one expert
// -- a whole expert at the usual prefill load of ~T*k/E rows, so each weight
// is dequantised once per call -- and 128 weight rows (gate/up: 64 gate
// rows and the same 64 up rows, so TIE's table SwiGLU
// (swiglu_activation_f32_f32_avx2) is applied to the accumulators in
// registers; down: two 64-row panels).  K advances 64 at a time through a
// double-buffered LDS pipeline: the global loads of step k+1 are issued
// into registers before the MFMAs of step k and written to the other buffer
// after them (the B tile dequantised from the panel layout on the way), one
// barrier per step.  Waves form a 4 (M) x 2 (N) grid of 64 x 64 tiles; the
// M index runs fastest across SIMDs, so a half-full tile still keeps every
// SIMD's matrix core busy.
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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int MT = MFMA_MT;   // pair rows per workgroup (256)
constexpr int NT = 128;       // weight rows per workgroup
constexpr int KS = 64;        // K per stage
constexpr int LDK = KS + 8;   // LDS row stride (bf16) -- padding against bank conflicts
constexpr int MF_THREADS = 512;

__device__ __forceinline__ uint16_t bf16_bits(float f)
{
	return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// two floats -> two round-to-nearest-even bf16 in one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16(float a, float b)
{
	const f32x2 v = {a, b};
	return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
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

// ------------------------------------------------------------------ roles
// Warp specialisation.  Waves 0-3 are consumers: they only issue MFMAs from
// the LDS tiles.  Waves 4-7 are producers: they fetch step k+2 from HBM,
// dequantise step k+1 and write it to the other LDS buffer while the
// consumers multiply step k.  One barrier per K-step joins the two.
//
// Producer thread pt = tid - 256 (0..255), per K-step of 64 values:
//   A (bf16 rows, 128 B): rows pt/8 + 32c (c < 8), 16-byte chunk pt%8, so a
//     wave instruction reads 8 whole 128-byte rows -- 8 cache lines, fully
//     used.  Split fp32 rows (256 B): rows pt/16 + 16c (c < 16), chunk pt%16.
//   B quantised: panel m = pt/128, panel row i = (pt/2)%64, half h = pt%2
//     (32 K values; the panel chunks are lane-contiguous already)
//   B bf16: B rows pt/8 + 32c (c < 4), chunk pt%8, like A
// Rows of A past the tile's end are neither loaded nor stored: MFMA output
// rows depend only on their own A row, and the epilogue drops those rows.
constexpr int N_CONSUMERS = 256;

template <bool SPLIT> struct Src {
	static constexpr int NA = SPLIT ? 16 : 8;
	const char *abase;     // activations + this thread's chunk offset
	uint32_t aoff[NA];     // byte offset of each A row; ~0u: past the tile
	const uint8_t *b[2];   // bf16: B rows (pt/8) of panels m = 0, 1; quantised: b[0] = panel row base
	size_t b32;            // bf16: bytes of 32 B rows
};

template <int TYPE, bool SPLIT> struct Pref {
	u32x4 a[SPLIT ? 16 : 8];
	u32x4 b[TYPE == TIE_GGML_Q6_K ? 4 : (TYPE == TIE_GGML_Q4_K ? 2 : 4)];
	uint32_t s6, d6; // Q6_K: the dword holding this thread's two scales, fp16 d
};

// B row in LDS of (panel m, panel row i).  Gate/up interleave the two
// matrices every 32 rows so that a consumer's two 32-column MFMA tiles hold
// the gate and the up values of the same F columns.
__device__ __forceinline__ int b_row(bool down, int m, int i)
{
	return down ? m * 64 + i : (i >> 5) * 64 + m * 32 + (i & 31);
}

// Workgroup barrier for the LDS pipeline: waits for this wave's LDS reads
// and writes only.  __syncthreads() would also wait for every global load
// in flight (vmcnt(0)), which would drain the prefetch pipeline each step.
__device__ __forceinline__ void lds_barrier()
{
	asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int TYPE, bool SPLIT>
__device__ __forceinline__ void load_step(const Src<SPLIT> &s, int pt, int kk, Pref<TYPE, SPLIT> &p)
{
	const size_t ak = (size_t)kk * KS * (SPLIT ? 4 : 2);
#pragma unroll
	for (int c = 0; c < Src<SPLIT>::NA; c++)
		if (s.aoff[c] != ~0u)
			p.a[c] = *reinterpret_cast<const u32x4 *>(s.abase + s.aoff[c] + ak);
	if constexpr (TYPE == TIE_GGML_BF16) {
#pragma unroll
		for (int c = 0; c < 4; c++)
			p.b[c] = *reinterpret_cast<const u32x4 *>(s.b[c >> 1] + (c & 1) * s.b32 + (size_t)kk * KS * 2 +
								   16 * (pt & 7));
	} else {
		const int i = (pt >> 1) & 63, h = pt & 1;
		const uint8_t *blk = s.b[0] + (size_t)(kk / 4) * panel_bytes(TYPE) + i * 16;
		if constexpr (TYPE == TIE_GGML_Q4_K) {
			// group g = kk%4: quant bytes 32g..32g+31 = chunks 1+2g, 2+2g; half h
			const int g = kk & 3;
			p.b[0] = *reinterpret_cast<const u32x4 *>(blk);
			p.b[1] = *reinterpret_cast<const u32x4 *>(blk + (1 + 2 * g + h) * 1024);
		} else {
			// half n = (kk/2)%2, quant row r = 2*(kk%2) + h (elements 32r + l)
			const int n = (kk >> 1) & 1, r = 2 * (kk & 1) + h;
			p.b[0] = *reinterpret_cast<const u32x4 *>(blk + (4 * n + 2 * (r & 1)) * 1024);
			p.b[1] = *reinterpret_cast<const u32x4 *>(blk + (4 * n + 2 * (r & 1) + 1) * 1024);
			p.b[2] = *reinterpret_cast<const u32x4 *>(blk + (8 + 2 * n) * 1024);
			p.b[3] = *reinterpret_cast<const u32x4 *>(blk + (9 + 2 * n) * 1024);
			p.s6 = *reinterpret_cast<const uint32_t *>(blk + 12 * 1024 + 4 * ((8 * n + 2 * r) >> 2));
			p.d6 = *reinterpret_cast<const uint16_t *>(blk - i * 16 + Q6K_CHUNKS * 1024 + 2 * i);
		}
	}
}

template <int TYPE, bool DOWN, bool SPLIT>
__device__ __forceinline__ void store_step(const Pref<TYPE, SPLIT> &p, const Src<SPLIT> &s, int pt, int kk,
					   uint16_t *__restrict__ As, uint16_t *__restrict__ Alo,
					   uint16_t *__restrict__ Bs)
{
	// A
#pragma unroll
	for (int c = 0; c < Src<SPLIT>::NA; c++) {
		if (s.aoff[c] == ~0u)
			continue;
		if (!SPLIT) {
			reinterpret_cast<u32x4 *>(As + ((pt >> 3) + 32 * c) * LDK)[pt & 7] = p.a[c];
		} else {
			const int o = ((pt >> 4) + 16 * c) * LDK + 4 * (pt & 15);
			const float v0 = __uint_as_float(p.a[c].x), v1 = __uint_as_float(p.a[c].y);
			const float v2 = __uint_as_float(p.a[c].z), v3 = __uint_as_float(p.a[c].w);
			const float hi0 = (float)(__bf16)v0, hi1 = (float)(__bf16)v1;
			const float hi2 = (float)(__bf16)v2, hi3 = (float)(__bf16)v3;
			*reinterpret_cast<u32x2 *>(As + o) = u32x2{pack_bf16(hi0, hi1), pack_bf16(hi2, hi3)};
			*reinterpret_cast<u32x2 *>(Alo + o) = u32x2{pack_bf16(v0 - hi0, v1 - hi1), pack_bf16(v2 - hi2, v3 - hi3)};
		}
	}
	// B
	const int m = pt >> 7, i = (pt >> 1) & 63, h = pt & 1;
	uint16_t *brow = Bs + b_row(DOWN, m, i) * LDK;
	if constexpr (TYPE == TIE_GGML_BF16) {
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<u32x4 *>(Bs + b_row(DOWN, c >> 1, (pt >> 3) + 32 * (c & 1)) * LDK)[pt & 7] = p.b[c];
	} else if constexpr (TYPE == TIE_GGML_Q4_K) {
		// sub-blocks 2g (low nibbles, K 0..31) and 2g+1 (high nibbles, K 32..63)
		const int g = kk & 3;
		const u32x4 c0 = p.b[0];
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
		const uint32_t qw[4] = {p.b[1].x, p.b[1].y, p.b[1].z, p.b[1].w};
		uint32_t lo[4], hi[4];
#pragma unroll
		for (int j = 0; j < 4; j++) {
			lo[j] = qw[j] & 0x0f0f0f0fu;
			hi[j] = (qw[j] >> 4) & 0x0f0f0f0fu;
		}
		// keep the masks byte-parallel so each weight is one v_cvt_f32_ubyteN
		asm volatile("" : "+v"(lo[0]), "+v"(lo[1]), "+v"(lo[2]), "+v"(lo[3]), "+v"(hi[0]), "+v"(hi[1]),
			     "+v"(hi[2]), "+v"(hi[3]));
		uint32_t pl[8], ph[8];
#pragma unroll
		for (int j = 0; j < 8; j++) {
			const uint32_t wl = lo[j >> 1], wh = hi[j >> 1];
			const int s0 = 16 * (j & 1);
			pl[j] = pack_bf16(__builtin_fmaf((float)((wl >> s0) & 0xffu), D0, M0),
					  __builtin_fmaf((float)((wl >> (s0 + 8)) & 0xffu), D0, M0));
			ph[j] = pack_bf16(__builtin_fmaf((float)((wh >> s0) & 0xffu), D1, M1),
					  __builtin_fmaf((float)((wh >> (s0 + 8)) & 0xffu), D1, M1));
		}
		uint16_t *d0 = brow + 16 * h; // low nibbles: K 16h..16h+15; high nibbles: 32+16h..
		reinterpret_cast<u32x4 *>(d0)[0] = u32x4{pl[0], pl[1], pl[2], pl[3]};
		reinterpret_cast<u32x4 *>(d0)[1] = u32x4{pl[4], pl[5], pl[6], pl[7]};
		reinterpret_cast<u32x4 *>(d0 + 32)[0] = u32x4{ph[0], ph[1], ph[2], ph[3]};
		reinterpret_cast<u32x4 *>(d0 + 32)[1] = u32x4{ph[4], ph[5], ph[6], ph[7]};
	} else {
		// Q6_K: q = (ql nibble | qh bits << 4); w = (d*sc) * (q - 32), exact in fp32
		const int n = (kk >> 1) & 1, r = 2 * (kk & 1) + h;
		const int sj = 8 * n + 2 * r;       // scale of l < 16; sj + 1 for l >= 16
		const float d = half_bits_to_float(p.d6);
		const float W0 = d * (float)(int8_t)((p.s6 >> (8 * (sj & 3))) & 0xffu);
		const float W1 = d * (float)(int8_t)((p.s6 >> (8 * ((sj + 1) & 3))) & 0xffu);
		const float N0 = -32.0f * W0, N1 = -32.0f * W1;
		const int nsh = 4 * (r >> 1), hsh = 2 * r;
		const uint32_t qlw[8] = {p.b[0].x, p.b[0].y, p.b[0].z, p.b[0].w, p.b[1].x, p.b[1].y, p.b[1].z, p.b[1].w};
		const uint32_t qhw[8] = {p.b[2].x, p.b[2].y, p.b[2].z, p.b[2].w, p.b[3].x, p.b[3].y, p.b[3].z, p.b[3].w};
		uint32_t qv[8];
#pragma unroll
		for (int j = 0; j < 8; j++)
			qv[j] = ((qlw[j] >> nsh) & 0x0f0f0f0fu) | (((qhw[j] >> hsh) & 0x03030303u) << 4);
		asm volatile("" : "+v"(qv[0]), "+v"(qv[1]), "+v"(qv[2]), "+v"(qv[3]), "+v"(qv[4]), "+v"(qv[5]),
			     "+v"(qv[6]), "+v"(qv[7]));
		uint32_t pk[16];
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const uint32_t wd = qv[j >> 1];
			const int s0 = 16 * (j & 1);
			const float W = j < 8 ? W0 : W1, N = j < 8 ? N0 : N1;
			pk[j] = pack_bf16(__builtin_fmaf((float)((wd >> s0) & 0xffu), W, N),
					  __builtin_fmaf((float)((wd >> (s0 + 8)) & 0xffu), W, N));
		}
		uint16_t *dst = brow + 32 * (r & 1);
#pragma unroll
		for (int c = 0; c < 4; c++)
			reinterpret_cast<u32x4 *>(dst)[c] = u32x4{pk[4 * c], pk[4 * c + 1], pk[4 * c + 2], pk[4 * c + 3]};
	}
}

__device__ __forceinline__ bf16x8 lds_frag(const uint16_t *base, int row, int k)
{
	return *reinterpret_cast<const bf16x8 *>(base + row * LDK + k);
}

// ------------------------------------------------------------------ kernel
template <int TYPE, bool DOWN, bool SPLIT, int NK>
__global__ __launch_bounds__(MF_THREADS) void mfma_experts_kernel(MfmaArgs a)
{
	// split activations need a second A tile: single-buffered then (that
	// path is HBM-bound, the extra barrier costs little)
	constexpr int NBUF = SPLIT ? 1 : 2;
	__shared__ __attribute__((aligned(16))) uint16_t As[NBUF][MT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Bs[NBUF][NT * LDK];
	__shared__ __attribute__((aligned(16))) uint16_t Alo[1][SPLIT ? MT * LDK : 8];

	// XCD-aware tile order.  Consecutive workgroup ids are spread round-robin
	// over the 8 XCDs, each with its own L2.  The id is remapped so that each
	// XCD takes a contiguous run of (tile, N-slab) work items; the N-slabs of
	// one expert tile then share an XCD and read the tile's gathered
	// activation rows from that XCD's L2 instead of from the MALL.
	const int nslab = gridDim.x;
	const int live = *a.ntiles * nslab;
	const int per_xcd = (live + 7) / 8;
	const int lin = blockIdx.y * gridDim.x + blockIdx.x;
	const int v = (lin % 8) * per_xcd + lin / 8;
	if (lin / 8 >= per_xcd || v >= live)
		return;
	const int tile = v / nslab;
	const int slab = v % nslab;
	const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
	const int pbase = a.offsets[e] + m0;
	const int nrows = min(MT, a.offsets[e + 1] - pbase);
	const int nk = NK > 0 ? NK : a.in / KS;
	const int w = threadIdx.x >> 6;

	if (threadIdx.x >= N_CONSUMERS) {
		// ---------------------------------------------------------- producer
		const int pt = threadIdx.x - N_CONSUMERS;
		Src<SPLIT> src;
		{
			constexpr int RPI = SPLIT ? 16 : 32; // rows per A instruction
			const int esz = SPLIT ? 4 : 2;
			src.abase = (SPLIT ? (const char *)a.a32 : (const char *)a.a16) + 16 * (pt % (64 / RPI * 4));
#pragma unroll
			for (int c = 0; c < Src<SPLIT>::NA; c++) {
				const int r = pt / (256 / RPI) + RPI * c;
				const int row = r < nrows ? (DOWN ? pbase + r : a.pairs[pbase + r] / a.k) : -1;
				src.aoff[c] = row < 0 ? ~0u : (uint32_t)((size_t)row * a.in * esz);
			}
		}
		if constexpr (TYPE == TIE_GGML_BF16) {
			src.b32 = (size_t)32 * a.in * 2;
#pragma unroll
			for (int mm = 0; mm < 2; mm++) {
				const int mat = DOWN ? 0 : mm;
				const int rt = DOWN ? 2 * slab + mm : slab;
				const uint8_t *base = a.w[mat] + (size_t)e * a.expert_bytes[mat];
				src.b[mm] = base + ((size_t)(rt * 64 + (pt >> 3)) * a.in) * 2;
			}
		} else {
			const int mm = pt >> 7;
			const int mat = DOWN ? 0 : mm;
			const int rt = DOWN ? 2 * slab + mm : slab;
			src.b[0] = a.w[mat] + (size_t)e * a.expert_bytes[mat] + (size_t)rt * (a.in / QK) * panel_bytes(TYPE);
			src.b[1] = nullptr;
			src.b32 = 0;
		}
		Pref<TYPE, SPLIT> p0, p1;
		load_step<TYPE, SPLIT>(src, pt, 0, p0);
		if (nk > 1)
			load_step<TYPE, SPLIT>(src, pt, 1, p1);
		store_step<TYPE, DOWN, SPLIT>(p0, src, pt, 0, As[0], Alo[0], Bs[0]);
		lds_barrier();
		auto body = [&](int kk, Pref<TYPE, SPLIT> &held, Pref<TYPE, SPLIT> &next) {
#ifndef TIE_EXP_NO_PLOAD
			if (kk + 2 < nk)
				load_step<TYPE, SPLIT>(src, pt, kk + 2, next);
#endif
			__builtin_amdgcn_sched_barrier(0);
			if (NBUF == 1)
				lds_barrier(); // consumers are reading the only buffer
#ifdef TIE_EXP_NO_PSTORE
			if (false)
#else
			if (kk + 1 < nk)
#endif
				store_step<TYPE, DOWN, SPLIT>(held, src, pt, kk + 1, As[NBUF == 2 ? (kk + 1) & 1 : 0], Alo[0],
							      Bs[NBUF == 2 ? (kk + 1) & 1 : 0]);
			lds_barrier();
		};
		if constexpr (NK > 0) {
#pragma unroll
			for (int kk = 0; kk < NK; kk += 2) {
				body(kk, p1, p0);
				if (kk + 1 < NK)
					body(kk + 1, p0, p1);
			}
		} else {
			for (int kk = 0; kk < nk; kk += 2) {
				body(kk, p1, p0);
				if (kk + 1 < nk)
					body(kk + 1, p0, p1);
			}
		}
		return;
	}

	// -------------------------------------------------------------- consumer
	// wave (wm, wn): M rows 64wm..+63 and 128+64wm..+63, N columns 64wn..+63
	const int lane = threadIdx.x & 63;
	const int wm = w >> 1, wn = w & 1;
	const int lr = lane & 31, lk = 8 * (lane >> 5);
	const bool live0 = 64 * wm < nrows, live1 = 128 + 64 * wm < nrows;
	f32x16 acc[2][4];
#pragma unroll
	for (int sl = 0; sl < 2; sl++)
#pragma unroll
		for (int t = 0; t < 4; t++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[sl][t][j] = 0.0f;

	auto compute = [&](int cur) {
		const uint16_t *A = As[cur], *B = Bs[cur], *AL = Alo[0];
#pragma unroll
		for (int s = 0; s < KS / 16; s++) {
			const bf16x8 b0 = lds_frag(B, 64 * wn + lr, 16 * s + lk);
			const bf16x8 b1 = lds_frag(B, 64 * wn + 32 + lr, 16 * s + lk);
#pragma unroll
			for (int sl = 0; sl < 2; sl++) {
				if (!(sl ? live1 : live0))
					continue;
				const int r0 = 128 * sl + 64 * wm + lr;
				const bf16x8 a0 = lds_frag(A, r0, 16 * s + lk);
				const bf16x8 a1 = lds_frag(A, r0 + 32, 16 * s + lk);
				acc[sl][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[sl][0], 0, 0, 0);
				acc[sl][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[sl][1], 0, 0, 0);
				acc[sl][2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[sl][2], 0, 0, 0);
				acc[sl][3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[sl][3], 0, 0, 0);
				if (SPLIT) {
					const bf16x8 l0 = lds_frag(AL, r0, 16 * s + lk);
					const bf16x8 l1 = lds_frag(AL, r0 + 32, 16 * s + lk);
					acc[sl][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l0, b0, acc[sl][0], 0, 0, 0);
					acc[sl][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l0, b1, acc[sl][1], 0, 0, 0);
					acc[sl][2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l1, b0, acc[sl][2], 0, 0, 0);
					acc[sl][3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l1, b1, acc[sl][3], 0, 0, 0);
				}
			}
		}
	};
	lds_barrier(); // step 0 staged
	for (int kk = 0; kk < nk; kk++) {
#ifndef TIE_EXP_NO_CONS
		compute(NBUF == 2 ? (kk & 1) : 0);
#endif
		if (NBUF == 1)
			lds_barrier();
		lds_barrier();
	}

	// D layout of v_mfma_f32_32x32x16: lane l, register j holds
	// row 8*(j/4) + 4*(l/32) + j%4, column l%32.
#pragma unroll
	for (int sl = 0; sl < 2; sl++) {
		if (!(sl ? live1 : live0))
			continue;
#pragma unroll
		for (int i = 0; i < 2; i++) {
#pragma unroll
			for (int j = 0; j < 16; j++) {
				const int mrow = 128 * sl + 64 * wm + 32 * i + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
				if (mrow >= nrows)
					continue;
				const int p = pbase + mrow;
				if (!DOWN) {
					// acc[..][2i]: gate, acc[..][2i+1]: up, of F column slab*64 + 32*wn + lr
					const int col = slab * 64 + 32 * wn + lr;
					const float hv = tie_swiglu(acc[sl][2 * i][j], acc[sl][2 * i + 1][j], a.silu);
					if (SPLIT)
						a.h32[(size_t)p * a.rows + col] = hv;
					else
						a.h16[(size_t)p * a.rows + col] = bf16_bits(hv);
				} else {
					const int pair = a.pairs[p];
					float *yr = a.y + (size_t)pair * a.rows + slab * 128 + 64 * wn + lr;
					yr[0] = acc[sl][2 * i][j];
					yr[32] = acc[sl][2 * i + 1][j];
				}
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

template <bool DOWN, bool SPLIT, int NK>
static void launch_nk(const MfmaArgs &a, int type, dim3 grid, hipStream_t s)
{
	if (type == TIE_GGML_Q4_K)
		hipLaunchKernelGGL((mfma_experts_kernel<TIE_GGML_Q4_K, DOWN, SPLIT, NK>), grid, dim3(MF_THREADS), 0, s, a);
	else if (type == TIE_GGML_Q6_K)
		hipLaunchKernelGGL((mfma_experts_kernel<TIE_GGML_Q6_K, DOWN, SPLIT, NK>), grid, dim3(MF_THREADS), 0, s, a);
	else
		hipLaunchKernelGGL((mfma_experts_kernel<TIE_GGML_BF16, DOWN, SPLIT, NK>), grid, dim3(MF_THREADS), 0, s, a);
}

// K = 2048 / 4096 (gate/up of the 30B / 235B shapes) and 768 / 1536 (down)
// get fully unrolled K loops; any other K runs the rolled loop.
template <bool DOWN, bool SPLIT>
static hipError_t launch_one(const MfmaArgs &a, int type, dim3 grid, hipStream_t s)
{
	switch (a.in / KS) {
	case 12:
		launch_nk<DOWN, SPLIT, 12>(a, type, grid, s);
		break;
	case 24:
		launch_nk<DOWN, SPLIT, 24>(a, type, grid, s);
		break;
	case 32:
		launch_nk<DOWN, SPLIT, 32>(a, type, grid, s);
		break;
	case 64:
		launch_nk<DOWN, SPLIT, 64>(a, type, grid, s);
		break;
	default:
		launch_nk<DOWN, SPLIT, 0>(a, type, grid, s);
	}
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
	// the kernels address activation rows with 32-bit byte offsets
	if ((size_t)T * L.d * 4 > 0xfffffffeu || (size_t)npairs * L.F * 4 > 0xfffffffeu)
		return hipErrorInvalidValue;
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
