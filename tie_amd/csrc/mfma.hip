// mfma.hip -- grouped expert GEMMs on the bf16 matrix cores (large T).
//
// Reference: TIE runs every (token, expert) pair as three GEMVs
// (process_expert_task, engine.c:916-964) with no reuse of an expert's
// weights across tokens.  For large T the pairs are grouped by expert
// (dispatch.hip) and each expert's weights are dequantised once per work
// tile and multiplied against all of the tile's tokens with
// v_mfma_f32_32x32x16_f16 (Q4_K / Q6_K weights) or _bf16 (BF16 weights):
//
//   gate/up:  G = X_e Wg_e^T, U = X_e Wu_e^T, h = silu_tab(G) * U  (fused)
//   down:     Y = h_e Wd_e^T, scattered to the pairs' rows of y
//
// Work tile: up to MT pair rows of one expert (MFMA_MT_GU = 160 for
// gate/up, MFMA_MT_GU_SMALL = 64 for gate/up with few pairs per expert,
// MFMA_MT_DN = 128 for down; an expert with more pairs is split
// evenly over several tiles) x 128 F columns (gate/up: of gate and of up)
// or 256 output columns (down).  A workgroup is 4 waves, one per SIMD;
// wave w owns two 32-wide column tiles -- gate/up: the gate and the up tile
// of F columns 32w..32w+31, so TIE's table SwiGLU
// (swiglu_activation_f32_f32_avx2) is applied to the accumulators in
// registers; down: columns 64w..64w+63 -- against all rows of the tile (up
// to MT/32 x 2 accumulator tiles of 32x32).
//
// Both operands are staged per K stage by direct global->LDS loads
// (global_load_lds_dwordx4) into double-buffered LDS tiles, one stage
// ahead: the activations (A, 16-bit rows gathered by pair) and, for Q4_K /
// Q6_K, the raw panel chunks of the workgroup's 4 weight panels (1 KiB
// each: the panel layout of common.h).  Quantised stages are 64 K: a Q4_K
// stage is one 64-weight group (scale chunk + 2 quant chunks); a Q6_K stage
// is quarters p and p + 2 of a 128-weight half, which share their ql / qh
// bytes (low / high nibbles, qh bits 2p and 2p + 4), so a stage needs 5
// chunks, and the activations' K order inside the stage is permuted to
// match.  Small stages and tiles keep a workgroup at about 64-75 KiB of LDS
// and 256 registers per lane: two workgroups share a CU (two waves per
// SIMD), so one's stalls and pipeline fill / drain overlap the other's
// MFMAs (the small-tile gate/up kernel: 40 KiB, 128 registers, three).  No register holds a prefetched stage, and the compiler's
// wait-count pass never sees (and never waits for) the prefetch: the stage
// barrier is the wait.  In the 32x32x16 B-operand layout a lane holds 8
// K values of one weight row -- 8 consecutive quant bytes of its lane-row
// in the panel (the activations' K order matches) -- which it reads from
// LDS and dequantises
// between the MFMAs: every weight of the tile is dequantised exactly once,
// and each B fragment feeds one MFMA per 32-row M tile (an f16 lane holds
// the pairs (0,2), (1,3), (4,6), (5,7) of those 8).  BF16 weights
// (already MFMA operands) are prefetched into registers instead (one wave
// per SIMD, 64-K stages).  An A fragment (1 KiB) feeds two MFMAs.
//
// Numerics: fp32 accumulation of 16-bit products.  Q4_K / Q6_K weights are
// dequantised with packed f16 math (code in the mantissa of 1024.0, exact
// subtraction, one v_pk_fma_f16 / v_pk_mul_f16 rounding) and carry a factor
// 2^F16_SHIFT, which the epilogues take out of the fp32 accumulators
// (exact); x is rounded to f16 and h is stored as f16(h * 2^-h_shift), with
// the layer's h_shift chosen at upload so its typical |h| sits near 2^2 (far
// from both ends of f16's range), both with the K order inside each 8-group
// 0,2,1,3,4,6,5,7 (the dequantised pairs' order).  A token whose x or scaled
// h leaves the f16 range (|v| >= 65504, or not finite) is
// listed by route_bucket_kernel / the gate/up epilogue and recomputed afterwards
// in TIE's exact arithmetic (decode.hip), which overwrites its output row.
// The expert outputs y of the quantised kernels are stored as
// f16(y * 2^-y_shift), the layer's y_shift chosen at upload so the typical
// |y| sits near 2^4 (an 11-bit significand: bf16's 8 bits were the largest
// error term of the path, 2^-9 relative); a token with a y outside the f16
// range is recomputed like one whose x or h is.  With BF16 expert
// weights (exact in bf16) the activations are split into a bf16 high part
// and a bf16 remainder, stored as two bf16 planes (x by route_bucket_kernel, h
// by the gate/up epilogue), two MFMAs per product; this keeps the products
// to ~16 mantissa bits; that path is HBM-bound, so the extra MFMA work is
// hidden, and its y stays fp32.
#include "common.h"
#include "route.h"

#include <type_traits>

namespace tie {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Q4_K K per stage (64: one 64-weight group), and waves per SIMD of the
// gate/up and down kernels
#ifndef TIE_Q4K_KST
#define TIE_Q4K_KST 64
#endif
// the same for the 32-row tile kernels (decode-sized batches); 128 halves
// their stage barriers but measured slower on the 30B shapes (T = 32:
// 0.1202 vs 0.1193 ms, T = 64: 0.1358 vs 0.1315 ms)
#ifndef TIE_Q4K_KST_TINY
#define TIE_Q4K_KST_TINY 64
#endif
// Q6_K K per stage: 128 (one block half), or 64 (quarters {p, p + 2} of a
// half, which share their ql / qh bytes; the activations' K order is
// permuted to match)
#ifndef TIE_Q6K_KST
#define TIE_Q6K_KST 64
#endif
// Q4_K gate/up on the f16 matrix cores (weights dequantised with packed f16
// math; 0 keeps bf16)
#ifndef TIE_MFMA_F16
#define TIE_MFMA_F16 1
#endif
// decode-sized batches: items (expert, slab) found without a scan (0: the
// scanned tile list, as for larger batches)
#ifndef TIE_MFMA_DIRECT
#define TIE_MFMA_DIRECT 1
#endif
// Tiles with at least this many 32-row M tiles run the cross-stage
// software pipeline (fewer: each stage self-contained; 4 measured 1.3%
// faster than 3 at 235B T=1024, the same elsewhere; 1 and 2 slower at
// decode-sized batches: 30B T=32 +3.4% / +0.3%, LFM2 T=32 +8.6% / +2.3%)
// Q4_K on the f16 matrix cores, 64-K stages: lane half h takes sub-block h
// of the stage's group (nibble h of all 32 code bytes), so a lane needs the
// scale factors of one sub-block, not two (0: both halves take both)
#ifndef TIE_MFMA_UH
#define TIE_MFMA_UH 1
#endif
// Q6_K 32-row tiles: the block's d applied once per 256-K block to a
// block accumulator (fp32) instead of to every dequantised weight (f16)
#ifndef TIE_MFMA_DFOLD
#define TIE_MFMA_DFOLD 1
#endif
// activation rows past the tile's own not moved into LDS
#ifndef TIE_MFMA_ASKIP
#define TIE_MFMA_ASKIP 1
#endif
// epilogue halves (16 rows) past the tile's rows skipped
#ifndef TIE_MFMA_EPI_SKIP
#define TIE_MFMA_EPI_SKIP 1
#endif
// Q4_K 32-row gate/up tiles (with TIE_MFMA_UH): the MFMAs take q sc
// (exact), d is applied per 256-K block to an fp32 block sum, and the
// minimum term by one MFMA per block over the routing's sub-block sums of
// the activations (Workspace::xsum), in place of the second packed FMA
// per weight pair
#ifndef TIE_MFMA_QFOLD
#define TIE_MFMA_QFOLD 1
#endif
#ifndef TIE_MFMA_PIPE_NMT
#define TIE_MFMA_PIPE_NMT 4
#endif
// VALU instructions placed between two MFMAs of a stage's last step
#ifndef TIE_MFMA_TAIL_VALU
#define TIE_MFMA_TAIL_VALU 12
#endif
#ifndef TIE_MFMA_GU_WPE
#define TIE_MFMA_GU_WPE 2
#endif
// workgroups (one wave per SIMD each) per CU of the tiny-tile kernels
#ifndef TIE_MFMA_TINY_GU_WPC
#define TIE_MFMA_TINY_GU_WPC 4
#endif
#ifndef TIE_TINY_SILU_GLOBAL
#define TIE_TINY_SILU_GLOBAL 1
#endif
#ifndef TIE_MFMA_TINY_DN_WPC
#define TIE_MFMA_TINY_DN_WPC 3
#endif
// BF16 weights: loaded into registers two stages ahead (1) or one (0)
#ifndef TIE_BF16_B3
#define TIE_BF16_B3 1
#endif
// waves per SIMD of the BF16-weight gate/up and down kernels (their weights
// prefetched into registers)
#ifndef TIE_MFMA_BF16_WPE
#define TIE_MFMA_BF16_WPE 2
#endif
#ifndef TIE_MFMA_BF16_DN_WPE
#define TIE_MFMA_BF16_DN_WPE 2
#endif
#ifndef TIE_MFMA_DN_WPE
#define TIE_MFMA_DN_WPE 2
#endif
constexpr int NWAVES = 4;
constexpr int MF_THREADS = 64 * NWAVES;
constexpr int GU_COLS = 32 * NWAVES; // gate/up: F columns per tile (128)
constexpr int DN_COLS = 64 * NWAVES; // down: output columns per tile (256)

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

__device__ __forceinline__ float f16_to_f32(uint32_t bits)
{
	// v_cvt_f32_f16: exact, binary16 denormals included (not flushed in this build)
	return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

struct MfmaArgs {
	const uint8_t *w[2];     // gate/up: gate, up tensors; down: down tensor (both)
	size_t expert_bytes[2];
	int rows, in;            // per expert: weight rows, K
	const uint16_t *a16;     // A as bf16 rows (gate/up: x [T][d] by token; down: h [P][F] by position)
	const uint16_t *a16lo;   // split mode: the bf16 remainder plane of A
	int k;                   // experts per token (token = pair / k)
	int E;                   // experts
	const int32_t *cnt;      // [E] pairs per expert
	const int32_t *bucket;   // [E][bstride] the expert's pair ids in token order
	int bstride;
	const float *silu;
	uint16_t *h16;           // gate/up out (bf16, by position)
	uint16_t *h16lo;         // gate/up out, split mode: bf16 remainder plane
	int h_f16;               // gate/up out: h as f16(h * h_scale), pair-permuted K order (quantised down)
	float h_scale;           // 2^-h_shift of the layer
	float y_scale;           // down out (f16 operands): 2^(h_shift - F16_SHIFT [- y_shift]) takes the factors out
				 // (y_shift only for f16 y)
	float *y;                // down out, fp32 rows: y [pair][d] (BF16 experts), out [token][rows] (dense matrices)
	uint16_t *y16;           // down out (quantised experts): y [pair][d] as f16(y 2^-y_shift)
	int mt_cap;              // pair rows per tile at most, below MT (0: MT; dense matrices at small T)
	int direct;              // 32-row tiles, T <= MFMA_DIRECT_T: item (expert, slab), h rows [E][MFMA_DIRECT_T]
	int32_t *tok_flag;       // [T] gate/up, h_f16: tokens whose h left the f16 range
	int32_t *fix_list;       //     are appended here (once each) ...
	int32_t *fix_count;      //     ... and counted
	const uint16_t *xsum;    // Q4_K 32-row gate/up tiles (QF): [T][2][in/32] sub-block sums of A, f16 high and
	                         // remainder parts
};

// Token t's activations do not fit the f16 operands: list it (once) for
// the exact recomputation that follows the forward.
__device__ __forceinline__ void flag_token(int32_t *flag, int32_t *list, int32_t *count, int t)
{
	if (atomicCAS(flag + t, 0, 1) == 0)
		list[atomicAdd(count, 1)] = t;
}

template <int TYPE, bool DOWN = false, int MTR = 0> struct Cfg {
	// pair rows per work tile at most (MTR: the small-tile gate/up kernel's)
	static constexpr int MT = MTR                    ? MTR
				  : TYPE == TIE_GGML_BF16 ? (DOWN ? MFMA_MT_DN_BF16 : MFMA_MT_GU_BF16)
				  : DOWN                  ? MFMA_MT_DN
							  : MFMA_MT_GU;
	static constexpr bool SPLIT = TYPE == TIE_GGML_BF16; // bf16 weights take activations as hi + lo planes
	// Q4_K / Q6_K weights: f16 operands (activations as f16 with the K order
	// inside each 8-group 0,2,1,3,4,6,5,7; weights scaled by 2^F16_SHIFT)
	static constexpr bool F16 = TIE_MFMA_F16 && (TYPE == TIE_GGML_Q4_K || TYPE == TIE_GGML_Q6_K);
	// K per stage (Q4_K optionally 64: one 64-weight group per stage)
	static constexpr int KST = SPLIT ? 64
				    : (TYPE == TIE_GGML_Q4_K ? (MTR == MFMA_MT_TINY ? TIE_Q4K_KST_TINY : TIE_Q4K_KST)
				       : TYPE == TIE_GGML_Q6_K ? TIE_Q6K_KST : 128);
	// Q6_K 64-K stages hold quarters p and p + 2 of a block half
	static constexpr bool APERM = TYPE == TIE_GGML_Q6_K && KST == 64;
	// Q4_K f16, 64-K stages: K step s, lane half h is sub-block h, positions
	// 8s .. 8s + 7 (TIE_MFMA_UH)
	static constexpr bool UH = TIE_MFMA_UH && TYPE == TIE_GGML_Q4_K && F16 && KST == 64;
	static constexpr int SPB = QK / KST;                 // stages per 256-weight block (quantised)
	static constexpr int NPL = SPLIT ? 2 : 1;            // activation planes
	static constexpr int RB = KST * 2;                   // bytes per A row, plane and stage
	static constexpr int CPR = RB / 16;                  // 16-byte slots per row
	static constexpr int RPI = 64 / CPR;                 // rows per wave DMA instruction
	static constexpr int NDMA = MT / (NWAVES * RPI);     // DMA instructions per wave, plane and stage
	static constexpr int A_TILE = MT * RB;               // bytes per plane
	static constexpr int ABUF = NPL * A_TILE;            // bytes per buffer
	static constexpr int NSTEP = KST / 16;               // MFMA K steps per stage
	// Quantised weights are staged through LDS too (panel chunks of the
	// stage, by direct loads): no registers hold the next stage's weights.
	// BF16 weights are prefetched into registers.
	static constexpr bool B_LDS = !SPLIT;
	static constexpr int NCH = TYPE == TIE_GGML_Q4_K ? 1 + KST / 32 : (KST == 64 ? 5 : 7); // 1 KiB chunks per panel and stage
	static constexpr int PB = NCH * 1024;                     // bytes per panel and stage
	static constexpr int BBUF = B_LDS ? 4 * PB + (TYPE == TIE_GGML_Q6_K ? 4 * 128 : 0) : 0; // + Q6_K d planes
	// weight stage buffers: three (the weights of stage s + 2 in flight
	// while stage s computes: an HBM round trip is longer than a stage)
	// where they fit the budget of two workgroups per CU, else two
	// workgroups per CU: the tiny-tile kernels TIE_MFMA_TINY_GU_WPC /
	// _DN_WPC, the small-tile gate/up kernels 3, the others 2
	static constexpr int WG_PER_CU = MTR == MFMA_MT_TINY ? (DOWN ? TIE_MFMA_TINY_DN_WPC : TIE_MFMA_TINY_GU_WPC)
					 : MTR && !DOWN ? 3
					 : DOWN         ? TIE_MFMA_DN_WPE
							: TIE_MFMA_GU_WPE;
	static constexpr int LDS_BUDGET = (160 * 1024) / WG_PER_CU;
	static constexpr int ROFF_BYTES = 4 * RPI * NWAVES * 16 + 4 * MT; // row offsets + pair ids
	// stage buffers (activations and weights; NS - 1 stages in flight): as
	// many as the LDS budget of WG_PER_CU workgroups per CU allows, up to 4
	// (quantised weights; BF16 weights go to registers: 2 activation buffers)
	static constexpr int NS = !B_LDS ? 2
				  : 4 * (ABUF + BBUF) + ROFF_BYTES <= LDS_BUDGET ? 4
				  : 3 * (ABUF + BBUF) + ROFF_BYTES <= LDS_BUDGET ? 3 : 2;
	static_assert(NWAVES == 4, "epilogue tile size");
	// DMA instructions one wave issues per weight stage (dma_b)
	static constexpr int B_DMA = NCH + (TYPE == TIE_GGML_Q6_K ? 1 : 0);
	static constexpr int LDS_A = NS * ABUF, LDS_B = B_LDS ? NS * BBUF : 0;
	// the f16 kernels' epilogue tiles (gate/up: after the 32 KiB SiLU
	// table) reuse the stage buffers; the dynamic LDS covers both
	// gate/up: TIE's SiLU table staged in LDS for the epilogue, except in
	// the 32-row tile kernels, where the table's 32 KiB would cost a
	// workgroup per CU (they read it from global memory, L2-resident)
	static constexpr bool SILU_LDS = !DOWN && !(MTR == MFMA_MT_TINY && TIE_TINY_SILU_GLOBAL);
	static constexpr int EPI_BYTES =
		(F16 && !SPLIT) ? (SILU_LDS ? 32768 : 0) + NWAVES * 16 * (DOWN ? 72 : 40) * 4 : 0;
	static constexpr int STAGE_BYTES = LDS_A + LDS_B > EPI_BYTES ? LDS_A + LDS_B : EPI_BYTES;
	// The slot of 16-byte chunk c of row r is c ^ swz(r): the rows of a
	// fragment read then spread over all LDS banks without row padding
	// (which the direct global->LDS loads cannot make).
	__device__ static int swz(int r) { return CPR == 8 ? (r >> 1) & 7 : r & 15; }
};

// ------------------------------------------------------------------ B registers
// One stage of one lane's two weight rows (j = 0, 1), straight from HBM.
//   lane l: row n = l%32 of the column tile, K half h = l/32 of each 16-K step
template <int TYPE> struct BRegs;
__device__ __forceinline__ uint32_t lds_addr(const void *p);
__device__ __forceinline__ void dma16(const void *g, uint32_t lds);
__device__ __forceinline__ void dma16s(const void *base, uint32_t voff, uint32_t lds);
// Quantised weights: lane half h holds whole 16-byte code chunks (chunk h
// of each pair), so the 32 lanes of a half read 32 consecutive rows' slots
// (no LDS bank conflict); step s takes bytes 8 (s % 2) .. of them.
template <> struct BRegs<TIE_GGML_Q4_K> {
	u32x4 q[2][2];  // per 64-weight group of the stage: quant chunk h of its two
	u32x4 sc[2];    // chunk 0: d, dmin, 12 scale bytes
};
template <> struct BRegs<TIE_GGML_Q6_K> {
	u32x4 ql[2][2]; // ql chunks 2c + h of the stage's ql slots, c < ql slots / 2
	u32x4 qh[2];    // qh chunk h of the half
	u32x2 sc[2];    // the half's 8 scales
	uint32_t d[2];  // fp16 d
};
template <> struct BRegs<TIE_GGML_BF16> {
	u32x4 w[2][4];  // K 16s+8h..+7 of the stage, s = 0..3
};

// The lane's two weight rows.  Quantised: the lane-row's 16-byte slot in
// block column 0 of its panel (block column kb is kb panels further), and
// for Q6_K the offset from that slot to the row's fp16 d in the panel's d
// plane.  BF16: the row start.
struct BSrc {
	const uint8_t *p[2];
	int dofs[2];
};

template <int TYPE>
__device__ __forceinline__ void load_b(const BSrc &s, int st, int h, BRegs<TYPE> &b)
{
	static_assert(TYPE == TIE_GGML_BF16, "quantised weights are staged through LDS");
	constexpr int KST = Cfg<TYPE>::KST;
#pragma unroll
	for (int j = 0; j < 2; j++)
#pragma unroll
		for (int q = 0; q < 4; q++)
			b.w[j][q] = *reinterpret_cast<const u32x4 *>(s.p[j] + ((size_t)st * KST + 16 * q + 8 * h) * 2);
}

// The stage's weight chunks of the workgroup's 4 panels -> LDS buffer B:
// panel p (gate/up: gate panels 0, 1 and up panels 2, 3 of the tile's 128
// columns; down: 4 panels of its 256 columns), chunk slot c, 1 KiB each.
// Q4_K slots: 0 scales, 1..4 the stage's quant chunks 1+4h..4+4h.  Q6_K
// slots: 0..3 ql chunks 4h..4h+3, 4, 5 qh chunks 8+2h, 9+2h, 6 the scales;
// then the 4 panels' d planes (128 B each).  h = st % 2 (the block half).
// Wave w moves items 4c + w (panel (4c + w) / NCH, slot (4c + w) % NCH);
// their bases and panel offsets are set once per tile (BDma).
template <int TYPE, int MTR = 0> struct BDma {
	static constexpr int NCH = Cfg<TYPE, false, MTR>::NCH;
	const uint8_t *base[NCH]; // expert base of the item's matrix (wave-uniform)
	uint32_t pofs[NCH];       // the item's panel row offset in the expert (wave-uniform)
	int slot[NCH];            // the item's LDS slot
	uint32_t lofs[NCH];       // the item's LDS offset in a B buffer
	uint32_t lane16;          // 16 * lane
	const uint8_t *dbase;     // Q6_K: expert base of panel w's matrix
	uint32_t dpofs;           // Q6_K: offset of panel w's d plane in its first block column
};

template <int TYPE, bool DOWN, int MTR = 0>
__device__ __forceinline__ void bdma_init(const MfmaArgs &a, int e, int slab, int w, BDma<TYPE, MTR> &d)
{
	using C = Cfg<TYPE, false, MTR>;
	const uint32_t pbytes = (uint32_t)panel_bytes(TYPE);
	const uint32_t nkb = (uint32_t)(a.in / QK);
#pragma unroll
	for (int c = 0; c < C::NCH; c++) {
		const int it = NWAVES * c + w; // NWAVES == 4 panels
		const int p = it / C::NCH, s = it % C::NCH;
		const int mat = DOWN ? 0 : p >> 1;
		const int rt = DOWN ? 4 * slab + p : 2 * slab + (p & 1);
		d.base[c] = a.w[mat] + (size_t)e * a.expert_bytes[mat];
		d.pofs[c] = (uint32_t)rt * nkb * pbytes;
		d.slot[c] = s;
		d.lofs[c] = (uint32_t)(p * C::PB + s * 1024);
	}
	d.lane16 = 16u * (threadIdx.x & 63);
	{
		const int mat = DOWN ? 0 : w >> 1;
		const int rt = DOWN ? 4 * slab + w : 2 * slab + (w & 1);
		d.dbase = a.w[mat] + (size_t)e * a.expert_bytes[mat];
		d.dpofs = (uint32_t)rt * nkb * pbytes + Q6K_CHUNKS * 1024;
	}
}

template <int TYPE, bool DOWN, int MTR = 0>
__device__ __forceinline__ void dma_b(const BDma<TYPE, MTR> &d, int slab, int st, int w, uint8_t *B)
{
	using C = Cfg<TYPE, false, MTR>;
	const int half = st & 1, part = st % C::SPB;
	const uint32_t kofs = (uint32_t)(st / C::SPB) * (uint32_t)panel_bytes(TYPE);
	const uint32_t lb = lds_addr(B);
#pragma unroll
	for (int c = 0; c < C::NCH; c++) {
		const int s = d.slot[c];
		int chunk;
		if constexpr (TYPE == TIE_GGML_Q4_K)
			chunk = s == 0 ? 0 : (C::NCH - 1) * part + s;
		else if constexpr (C::APERM) {
			// ql chunks of quarters q, q + 2 of half n; the half's qh; scales
			const int n = (st >> 1) & 1, q = st & 1;
			chunk = s < 2 ? 4 * n + 2 * q + s : (s < 4 ? 8 + 2 * n + (s - 2) : 12);
		} else
			chunk = s < 4 ? 4 * half + s : (s < 6 ? 8 + 2 * half + (s - 4) : 12);
		dma16s(d.base[c], d.lane16 + (d.pofs[c] + kofs + (uint32_t)chunk * 1024),
		       __builtin_amdgcn_readfirstlane(lb + d.lofs[c]));
	}
	if constexpr (TYPE == TIE_GGML_Q6_K) {
		// the d plane of panel w (128 B)
		if ((threadIdx.x & 63) < 8)
			dma16s(d.dbase, d.lane16 + (d.dpofs + kofs), __builtin_amdgcn_readfirstlane(lb + 4 * C::PB + w * 128));
	}
}

// The lane's weights of the stage from LDS buffer B: row j of the lane in
// panel p[j], slot i[j].
template <int TYPE, int MTR = 0>
__device__ __forceinline__ void lds_b(const uint8_t *B, const int p[2], const int i[2], int st, int h, BRegs<TYPE> &b)
{
	using C = Cfg<TYPE, false, MTR>;
#pragma unroll
	for (int j = 0; j < 2; j++) {
		const uint8_t *pb = B + p[j] * C::PB + i[j] * 16;
		if constexpr (TYPE == TIE_GGML_Q4_K && C::UH) {
			// both code chunks of the stage's group (the lane half takes its nibble)
			b.q[j][0] = *reinterpret_cast<const u32x4 *>(pb + 1024);
			b.q[j][1] = *reinterpret_cast<const u32x4 *>(pb + 2 * 1024);
			b.sc[j] = *reinterpret_cast<const u32x4 *>(pb);
		} else if constexpr (TYPE == TIE_GGML_Q4_K) {
#pragma unroll
			for (int g = 0; g < (C::NCH - 1) / 2; g++)
				b.q[j][g] = *reinterpret_cast<const u32x4 *>(pb + (1 + 2 * g + h) * 1024);
			b.sc[j] = *reinterpret_cast<const u32x4 *>(pb);
		} else if constexpr (TYPE == TIE_GGML_Q6_K) {
			constexpr int NQL = C::APERM ? 2 : 4; // ql chunk slots
#pragma unroll
			for (int c = 0; c < NQL / 2; c++)
				b.ql[j][c] = *reinterpret_cast<const u32x4 *>(pb + (2 * c + h) * 1024);
			b.qh[j] = *reinterpret_cast<const u32x4 *>(pb + (NQL + h) * 1024);
			const int half = C::APERM ? (st >> 1) & 1 : st & 1;
			b.sc[j] = *reinterpret_cast<const u32x2 *>(pb + (NQL + 2) * 1024 + 8 * half);
			b.d[j] = *reinterpret_cast<const uint16_t *>(B + 4 * C::PB + p[j] * 128 + 2 * i[j]);
		}
	}
}

// the lane's half of the wave (its K half of each 16-K step)
__device__ __forceinline__ int lane_half()
{
	return (threadIdx.x >> 5) & 1;
}

// 8 weight codes (bytes of lo, hi) -> bf16x8 of fma(q, D, M)
__device__ __forceinline__ bf16x8 deq8(uint32_t lo, uint32_t hi, float D, float M)
{
	// keep the words byte-parallel so each weight is one v_cvt_f32_ubyteN
	asm volatile("" : "+v"(lo), "+v"(hi));
	u32x4 r;
	r.x = pack_bf16(__builtin_fmaf((float)(lo & 0xffu), D, M), __builtin_fmaf((float)((lo >> 8) & 0xffu), D, M));
	r.y = pack_bf16(__builtin_fmaf((float)((lo >> 16) & 0xffu), D, M), __builtin_fmaf((float)(lo >> 24), D, M));
	r.z = pack_bf16(__builtin_fmaf((float)(hi & 0xffu), D, M), __builtin_fmaf((float)((hi >> 8) & 0xffu), D, M));
	r.w = pack_bf16(__builtin_fmaf((float)((hi >> 16) & 0xffu), D, M), __builtin_fmaf((float)(hi >> 24), D, M));
	return __builtin_bit_cast(bf16x8, r);
}

// Q4_K 6-bit scale / min of sub-block j from the 12 scale bytes s[0..11]
// (words y, z, w of chunk 0), without branches (j is wave-uniform but not a
// constant; branches would split the schedule).  With i = j % 4:
//   j < 4:  sc = s[j] & 63,                       m = s[j+4] & 63
//   j >= 4: sc = s[j+4] & 15 | (s[j-4] >> 6) << 4, m = s[j+4] >> 4 | (s[j] >> 6) << 4
// s[j] / s[j+4] (j < 4) are byte i of y / z; s[j-4], s[j], s[j+4] (j >= 4)
// byte i of y, z, w.  The high parts' width is 0 for j < 4.
__device__ __forceinline__ void q4k_scale_min(const u32x4 &c0, int j, uint32_t &sc, uint32_t &mn)
{
	const bool hi = j >= 4;
	const uint32_t o = 8u * (uint32_t)(j & 3);
	const uint32_t wlo = hi ? 4u : 6u, whi = hi ? 2u : 0u;
	const uint32_t a = hi ? c0.w : c0.y, b = hi ? c0.w : c0.z;
	sc = __builtin_amdgcn_ubfe(a, o, wlo) | (__builtin_amdgcn_ubfe(c0.y, o + 6u, whi) << 4);
	mn = __builtin_amdgcn_ubfe(b, o + (hi ? 4u : 0u), wlo) | (__builtin_amdgcn_ubfe(c0.z, o + 6u, whi) << 4);
}

// Per-row dequantisation factors of the current 64-K group (Q4_K: scale D
// and offset M of its two sub-blocks) or stage (Q6_K: d).
struct Fac {
	float D[2][2], M[2][2]; // [row][sub-block]
	float d6[2];
};

// Q4_K: group g = 2*(st%2) + gi of the block; sub-blocks 2g (low nibbles,
// K 0..31 of the group) and 2g+1 (high nibbles, K 32..63).
template <int TYPE, int MTR = 0>
__device__ __forceinline__ void group_factors(const BRegs<TYPE> &b, int st, int gi, Fac &f)
{
#pragma unroll
	for (int j = 0; j < 2; j++) {
		if constexpr (TYPE == TIE_GGML_Q4_K) {
			const int g = (4 / Cfg<TYPE, false, MTR>::SPB) * (st % Cfg<TYPE, false, MTR>::SPB) + gi;
			const float d = f16_to_f32(b.sc[j].x & 0xffffu), dmin = f16_to_f32(b.sc[j].x >> 16);
#pragma unroll
			for (int u = 0; u < 2; u++) {
				uint32_t sc, mn;
				q4k_scale_min(b.sc[j], 2 * g + u, sc, mn);
				f.D[j][u] = d * (float)sc;
				f.M[j][u] = -(dmin * (float)mn);
			}
		} else if constexpr (TYPE == TIE_GGML_Q6_K) {
			f.d6[j] = f16_to_f32(b.d[j]);
		}
	}
}

// f16 path: weights carry a factor 2^F16_SHIFT so that the per-sub-block
// scales D (d * sc, as small as 2^-24 * 63) and the weights stay in f16's
// normal range; the gate/up epilogue takes the factor out (exact).
constexpr int F16_SHIFT = 8;

struct Fac16 {
	f16x2 SN[2][2]; // [row][sub-block]: (sc, -1024 sc), or (sc / 16, -64 sc) for the high nibbles
	f16x2 DM[2][2]; // [row][sub-block]: (d * 2^S, M * 2^S), M = -dmin * m
};

__device__ __forceinline__ f16x2 splat16(float v)
{
	const _Float16 h = (_Float16)v;
	return f16x2{h, h};
}

// In packed f16, exactly: the sub-block's 6-bit (sc, m) (in the mantissa
// of 1024.0, minus 1024), (sc, -1024 sc) (low nibbles) or (sc / 16, -64 sc)
// (high nibbles, which the dequantisation holds as 16 q), and d * 2^S; then
// M = -dmin * m * 2^S, rounded once.  The weight is then
// (q sc) d 2^S + M with q sc exact and one rounding (deq_step16), not
// q (d sc) + M with d sc rounded to f16 first: that rounding, shared by the
// 32 weights of a sub-block, was half of the weights' error.
template <int TYPE, int MTR = 0>
__device__ __forceinline__ void group_factors16(const BRegs<TYPE> &b, int st, int gi, Fac16 &f)
{
	const f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
	const f16x2 sn0 = {(_Float16)1.0f, (_Float16)(-1024.0f)};
	const f16x2 sn1 = {(_Float16)(1.0f / 16), (_Float16)(-64.0f)};
	const f16x2 sdm = {(_Float16)(float)(1 << F16_SHIFT), (_Float16)(-(float)(1 << F16_SHIFT))};
	if constexpr (Cfg<TYPE, false, MTR>::UH) {
		// the lane half's sub-block 2g + h only, into [j][0]
		const int h = lane_half();
		const f16x2 sn = h ? sn1 : sn0;
		const int g = st % Cfg<TYPE, false, MTR>::SPB;
#pragma unroll
		for (int j = 0; j < 2; j++) {
			const f16x2 dd = __builtin_bit_cast(f16x2, b.sc[j].x);
			uint32_t sc, mn;
			q4k_scale_min(b.sc[j], 2 * g + h, sc, mn);
			const f16x2 sm = __builtin_bit_cast(f16x2, (sc | (mn << 16)) | 0x64006400u) - k1024;
			f.SN[j][0] = f16x2{sm[0], sm[0]} * sn;
			f.DM[j][0] = f16x2{(_Float16)1.0f, sm[1]} * dd * sdm;
		}
		return;
	}
#pragma unroll
	for (int j = 0; j < 2; j++) {
		const int g = (4 / Cfg<TYPE, false, MTR>::SPB) * (st % Cfg<TYPE, false, MTR>::SPB) + gi;
		// (component x: this clang's __builtin_bit_cast of any other vector
		// component reads component x -- copy such a one to a scalar first)
		const f16x2 dd = __builtin_bit_cast(f16x2, b.sc[j].x);
#pragma unroll
		for (int u = 0; u < 2; u++) {
			uint32_t sc, mn;
			q4k_scale_min(b.sc[j], 2 * g + u, sc, mn);
			const f16x2 sm = __builtin_bit_cast(f16x2, (sc | (mn << 16)) | 0x64006400u) - k1024;
			f.SN[j][u] = f16x2{sm[0], sm[0]} * (u ? sn1 : sn0);
			f.DM[j][u] = f16x2{(_Float16)1.0f, sm[1]} * dd * sdm;
		}
	}
}
// The masks and the magic live in VGPRs (K16): a GFX9 VOP3 instruction takes
// no literal, so only then is each pair one v_and_or_b32.
struct K16 {
	uint32_t lo, hi, magic, q6, uh; // uh: the lane half's nibble mask (lo or hi)
};

__device__ __forceinline__ K16 k16_consts()
{
	K16 k = {0x000f000fu, 0x00f000f0u, 0x64006400u, 0x003f003fu, lane_half() ? 0x00f000f0u : 0x000f000fu};
	asm volatile("" : "+v"(k.lo), "+v"(k.hi), "+v"(k.magic), "+v"(k.q6), "+v"(k.uh));
	return k;
}

// The minimum term's factors of one weight row's block (its scale chunk
// c0): f16 -dmin m_sb 2^S for sub-blocks sb = 0..7 (element sb), each rounded
// once (m_sb dmin 2^S; dmin 2^S exact)
__device__ __forceinline__ f16x8 q4k_mins16(const u32x4 &c0)
{
	const uint32_t x = c0.x, z = c0.z, w = c0.w;
	const f16x2 dd = __builtin_bit_cast(f16x2, x);
	const _Float16 nd = dd[1] * (_Float16)(-(float)(1 << F16_SHIFT));
	const f16x2 ndm = {nd, nd};
	const f16x2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
	// m_0..3: bits 0-5 of the bytes of z; m_4..7: the high nibbles of w's
	// bytes and bits 6-7 of z's
	const uint32_t m03 = z & 0x3f3f3f3fu;
	const uint32_t m47 = ((w >> 4) & 0x0f0f0f0fu) | ((z >> 2) & 0x30303030u);
	const uint32_t pr[4] = {__builtin_amdgcn_perm(0u, m03, 0x0c010c00u), __builtin_amdgcn_perm(0u, m03, 0x0c030c02u),
				__builtin_amdgcn_perm(0u, m47, 0x0c010c00u), __builtin_amdgcn_perm(0u, m47, 0x0c030c02u)};
	f16x2 m[4];
#pragma unroll
	for (int i = 0; i < 4; i++)
		m[i] = (__builtin_bit_cast(f16x2, pr[i] | 0x64006400u) - k1024) * ndm;
	return f16x8{m[0][0], m[0][1], m[1][0], m[1][1], m[2][0], m[2][1], m[3][0], m[3][1]};
}

template <bool UH, bool QS = false> // QS: q sc only (exact), without d and M
__device__ __forceinline__ void deq_step16(const BRegs<TIE_GGML_Q4_K> &b, const Fac16 &f, const K16 &kc, int s,
					   f16x8 out[2])
{
	if constexpr (UH) {
		// step s: code bytes 8s .. 8s + 7 of the group (chunk s/2), the lane
		// half's nibble, its sub-block's factors
#pragma unroll
		for (int j = 0; j < 2; j++) {
			const u32x4 q4 = b.q[j][s >> 1];
			const u32x2 q = (s & 1) ? u32x2{q4.z, q4.w} : u32x2{q4.x, q4.y};
			const uint32_t w[4] = {q.x, q.x >> 8, q.y, q.y >> 8};
			const f16x2 sn = f.SN[j][0], dm = f.DM[j][0];
			f16x2 r[4];
#pragma unroll
			for (int i = 0; i < 4; i++) {
				// v = 1024 + q (low nibbles) or 1024 + 16 q (high); q sc exact
				const f16x2 v = __builtin_bit_cast(f16x2, (w[i] & kc.uh) | kc.magic);
				const f16x2 qs = __builtin_elementwise_fma(v, f16x2{sn[0], sn[0]}, f16x2{sn[1], sn[1]});
				if constexpr (QS)
					r[i] = qs;
				else
					r[i] = __builtin_elementwise_fma(qs, f16x2{dm[0], dm[0]}, f16x2{dm[1], dm[1]});
			}
			out[j] = f16x8{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
		}
		return;
	}
#pragma unroll
	for (int j = 0; j < 2; j++) {
		// step s of the stage: 64-weight group gi = s / 4 (stages of 128 K
		// hold two), quarter sub = s % 4
		const int gi = s >> 2, sub = s & 3, u = sub >> 1;
		const u32x4 q4 = b.q[j][gi];
		const u32x2 q = (sub & 1) ? u32x2{q4.z, q4.w} : u32x2{q4.x, q4.y};
		const uint32_t msk = u ? kc.hi : kc.lo;
		uint32_t w[4] = {q.x, q.x >> 8, q.y, q.y >> 8};
		f16x2 r[4];
#pragma unroll
		for (int i = 0; i < 4; i++) {
			// v = 1024 + q (low nibbles) or 1024 + 16 q (high); q sc exact
			const f16x2 v = __builtin_bit_cast(f16x2, (w[i] & msk) | kc.magic);
			const f16x2 sn = f.SN[j][u], dm = f.DM[j][u];
			const f16x2 qs = __builtin_elementwise_fma(v, f16x2{sn[0], sn[0]}, f16x2{sn[1], sn[1]});
			r[i] = __builtin_elementwise_fma(qs, f16x2{dm[0], dm[0]}, f16x2{dm[1], dm[1]});
		}
		out[j] = f16x8{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
	}
}

// Dequantise the B fragments of 16-K step s of stage st for both rows.
// Q4_K: step s is in group gi = s/4; steps 0, 1 of a group take the low
// nibbles of bytes 0..7, 8..15 of the lane half's chunk h, steps 2, 3 the
// high nibbles (positions 16h + 8(s%2) + i of the sub-block).  Q6_K: step
// s is quarter r of the stage's half, positions l = 16h + 8(s%2) + i (bytes
// 8(s%2) .. of ql / qh chunk h), code q = ql nibble | qh bits << 4 with
// scale 8*half + l/16 + 2r (TIE's block_q6_k).
template <int TYPE>
__device__ __forceinline__ void deq_step(const BRegs<TYPE> &b, const Fac &f, int st, int s, bf16x8 out[2])
{
#pragma unroll
	for (int j = 0; j < 2; j++) {
		if constexpr (TYPE == TIE_GGML_BF16) {
			out[j] = __builtin_bit_cast(bf16x8, b.w[j][s]);
		} else if constexpr (TYPE == TIE_GGML_Q4_K) {
			const int gi = s >> 2, sub = s & 3, u = sub >> 1;
			const u32x4 q4 = b.q[j][gi];
			const u32x2 q = (sub & 1) ? u32x2{q4.z, q4.w} : u32x2{q4.x, q4.y};
			out[j] = deq8((q.x >> (4 * u)) & 0x0f0f0f0fu, (q.y >> (4 * u)) & 0x0f0f0f0fu, f.D[j][u], f.M[j][u]);
		} else {
			// quarter r; 64-K stages: quarter p for steps 0, 1 and p + 2 for 2, 3
			const int r = Cfg<TYPE>::APERM ? (st & 1) + 2 * (s >> 1) : s >> 1, lh = s & 1;
			const u32x4 ql4 = b.ql[j][Cfg<TYPE>::APERM ? 0 : r & 1], qh4 = b.qh[j];
			const u32x2 ql = lh ? u32x2{ql4.z, ql4.w} : u32x2{ql4.x, ql4.y};
			const u32x2 qh = lh ? u32x2{qh4.z, qh4.w} : u32x2{qh4.x, qh4.y};
			const int nsh = 4 * (r >> 1), hsh = 2 * r;
			const uint32_t lo = ((ql.x >> nsh) & 0x0f0f0f0fu) | (((qh.x >> hsh) & 0x03030303u) << 4);
			const uint32_t hi = ((ql.y >> nsh) & 0x0f0f0f0fu) | (((qh.y >> hsh) & 0x03030303u) << 4);
			// scale 2r + h: positions 16 h + 8 (s % 2) + i of the quarter
			const uint32_t sw = r < 2 ? b.sc[j].x : b.sc[j].y;
			const float W = f.d6[j] * (float)(int8_t)((sw >> (16 * (r & 1) + 8 * lane_half())) & 0xffu);
			out[j] = deq8(lo, hi, W, -32.0f * W);
		}
	}
}

// Q6_K step s in f16: the step's 8 six-bit codes of the lane's row (bytes of
// lo, hi, as in deq_step) -> f16 pairs (K 0,2), (1,3), (4,6), (5,7): a code
// in the mantissa of 1024.0, minus 1056 = code - 32 (exact), times
// d * sc * 2^F16_SHIFT (v_pk_mul_f16, one rounding).
template <bool NOD = false> // NOD: without the factor d 2^S ((q - 32) sc, exact)
__device__ __forceinline__ void deq_step16_q6k(const BRegs<TIE_GGML_Q6_K> &b, const Fac &f, const K16 &kc, int st, int s,
					       f16x8 out[2])
{
	const f16x2 k1056 = {(_Float16)1056.0f, (_Float16)1056.0f};
#pragma unroll
	for (int j = 0; j < 2; j++) {
		const int r = Cfg<TIE_GGML_Q6_K>::APERM ? (st & 1) + 2 * (s >> 1) : s >> 1, lh = s & 1;
		const u32x4 ql4 = b.ql[j][Cfg<TIE_GGML_Q6_K>::APERM ? 0 : r & 1], qh4 = b.qh[j];
		const u32x2 ql = lh ? u32x2{ql4.z, ql4.w} : u32x2{ql4.x, ql4.y};
		const u32x2 qh = lh ? u32x2{qh4.z, qh4.w} : u32x2{qh4.x, qh4.y};
		const int nsh = 4 * (r >> 1), hsh = 2 * r;
		// the code bytes' bits 6, 7 may hold other qh bits: the f16 pairs
		// below keep 6 bits of each (kc.q6), so a rotate (bits 2 hsh.. of
		// each qh byte to bits 4, 5) and one bit-field insert per word put
		// the qh field above the ql nibble
		auto qhs = [&](uint32_t v) { return __builtin_amdgcn_alignbit(v, v, (uint32_t)(hsh + 28) & 31u); };
		const uint32_t lo = ((ql.x >> nsh) & 0x0f0f0f0fu) | (qhs(qh.x) & 0xf0f0f0f0u);
		const uint32_t hi = ((ql.y >> nsh) & 0x0f0f0f0fu) | (qhs(qh.y) & 0xf0f0f0f0u);
		// scale 2r + h: positions 16 h + 8 (s % 2) + i of the quarter
		const uint32_t sw = r < 2 ? b.sc[j].x : b.sc[j].y;
		// (q - 32) sc exact in f16 (|sc| <= 64: |(q - 32) sc| <= 2048), then
		// times d 2^S with one rounding: d sc is not rounded to f16 first
		const f16x2 SC = splat16((float)(int8_t)((sw >> (16 * (r & 1) + 8 * lane_half())) & 0xffu));
		const f16x2 D = splat16(f.d6[j] * (float)(1 << F16_SHIFT));
		const uint32_t w[4] = {lo, lo >> 8, hi, hi >> 8};
		f16x2 q[4];
#pragma unroll
		for (int i = 0; i < 4; i++) {
			q[i] = (__builtin_bit_cast(f16x2, (w[i] & kc.q6) | kc.magic) - k1056) * SC;
			if constexpr (!NOD)
				q[i] = q[i] * D;
		}
		out[j] = f16x8{q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
	}
}

// ------------------------------------------------------------------ A staging
// A stage: up to MT rows x KST K of each plane, RB bytes per row.  Direct
// global->LDS loads (global_load_lds_dwordx4): one wave instruction writes
// 64 consecutive 16-byte LDS slots = RPI whole rows; lane l fills slot l%CPR
// of row l/CPR with the row's chunk slot ^ swz(row).  Wave w, instruction c
// covers rows RPI*(NWAVES c + w) ..; swz(row) does not depend on c.  Only
// the rows of the tile's live 32-row M tiles are loaded.
// The byte offsets of the tile's rows sit in an LDS table written once per
// tile, not in registers, ordered so that the NDMA offsets one lane needs
// per stage are contiguous (one wait per stage).  Rows of a live M tile past
// the tile's end read the tile's first row instead (no branch; an MFMA
// output row depends only on its own A row, and the epilogue drops those
// rows).
constexpr int ROFF_STRIDE = 16; // offsets per lane slot (>= NDMA, multiple of 4)
struct ASrc {
	const char *base[2];   // planes (wave-uniform)
	uint32_t cofs;         // this lane's chunk offset in a row
	const uint32_t *roff;  // LDS: this lane's ROFF_STRIDE row byte offsets
	int nrows;             // the tile's rows (wave-uniform)
};

// The LDS offset of a generic pointer into LDS: a flat LDS address is the
// shared aperture's base in the high 32 bits and the offset in the low 32,
// so truncation gives the offset (a cast to the LDS address space would add
// a null-pointer test: a 64-bit compare and select per address).
__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
	return (uint32_t)(uintptr_t)p;
}

// 16 bytes from global memory to LDS address lds + 16 * lane.  Issued as
// inline asm so that the compiler's wait-count pass does not order the
// fragment reads of the other buffer after it; the stage barrier waits for it.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds)
{
	asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// The same from a wave-uniform base (SGPR pair) plus a 32-bit per-lane byte
// offset: no 64-bit address arithmetic per load.
__device__ __forceinline__ void dma16s(const void *base, uint32_t voff, uint32_t lds)
{
	asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
		     : "memory", "m0");
}

// Only the rows of the NMT live 32-row M tiles are moved (the fragments of
// the other rows are never read).
template <int TYPE, bool DOWN, int NMT, int MTR>
__device__ __forceinline__ void dma_a(const ASrc &s, int st, int w, const uint8_t *buf)
{
	using C = Cfg<TYPE, DOWN, MTR>;
	constexpr int NLIVE = (32 * NMT + NWAVES * C::RPI - 1) / (NWAVES * C::RPI); // DMA instructions per wave and plane
	static_assert(NLIVE <= C::NDMA, "live rows exceed the tile");
	// byte offset of the stage in an A row (APERM: block, half, quarter p;
	// the lane's chunk offset covers the quarter p + 2 part)
	const uint32_t ko = C::APERM ? 512u * (st >> 2) + 256u * ((st >> 1) & 1) + 64u * (st & 1) : (uint32_t)st * C::RB;
	uint32_t off[(C::NDMA + 3) / 4 * 4]; // whole 16-byte reads (the lane slot holds ROFF_STRIDE entries)
	static_assert(C::NDMA <= ROFF_STRIDE, "row offset slot too small");
#pragma unroll
	for (int c = 0; c < NLIVE; c += 4)
		*reinterpret_cast<u32x4 *>(off + c) = *reinterpret_cast<const u32x4 *>(s.roff + c);
	const uint32_t lk = s.cofs + ko;
#pragma unroll
	for (int pl = 0; pl < C::NPL; pl++)
#pragma unroll
		for (int c = 0; c < NLIVE; c++) {
			const int r0 = C::RPI * (NWAVES * c + w);
			// rows past the tile's are not moved (their fragments feed only
			// output rows that are never stored); with two stage buffers every
			// stage barrier waits for all loads, so the skipped ones change no
			// wait count
			if (TIE_MFMA_ASKIP && C::NS == 2 && r0 >= s.nrows)
				continue;
			const uint32_t dst = lds_addr(buf + pl * C::A_TILE + r0 * C::RB);
			dma16s(s.base[pl], off[c] + lk, __builtin_amdgcn_readfirstlane(dst));
		}
}

// Waits for this wave's global loads (the weights and the DMA of the next
// stage) and LDS reads, then joins the workgroup.  Issued through the
// builtins, not inline asm: the compiler's wait-count pass then knows that
// every older load has landed, and inserts no wait inside the next stage
// for the weights prefetched here (such a wait would also drain the
// prefetch issued at that stage's start, which the pass cannot see).
__device__ __forceinline__ void stage_barrier()
{
	__builtin_amdgcn_s_waitcnt(0); // vmcnt(0) expcnt(0) lgkmcnt(0)
	__builtin_amdgcn_s_barrier();
}

// Cycle accounting of the matrix-core kernels (diagnostic builds only:
// -DTIE_MFMA_TRACE): summed over workgroups (wave 0 of each), [down][0]
// cycles in run_tile, [1] in stage barriers, [2] in the epilogue, [3]
// workgroups, [4] cycles from kernel entry to the tile's start (the tile
// mapping); read by tie_hip_debug_mfma_trace.
#ifdef TIE_MFMA_TRACE
__device__ unsigned long long g_mfma_trace[2][8];
#endif
#ifdef TIE_MFMA_TIMELINE
// diagnostic timeline: [down][workgroup] = {start, end} (s_memrealtime,
// 100 MHz) of each live workgroup of the last launch
constexpr int MFMA_TL_WG = 16384;
__device__ unsigned long long g_mfma_tl[2][MFMA_TL_WG][2];
#endif

// The same, but the N youngest vector loads (the next-but-one weight
// stage's DMA, issued last) may stay in flight: loads complete in order, so
// everything older has landed.  N < 64 (expcnt and lgkmcnt 0).
template <int N> __device__ __forceinline__ void stage_barrier_keep()
{
	static_assert(N >= 0 && N < 64, "vmcnt field");
	// gfx9 s_waitcnt: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8
	__builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14));
	__builtin_amdgcn_s_barrier();
}

// Operand arithmetic of a quantised kernel: bf16 fragments, or f16 ones
// (Q4_K gate/up).
template <int TYPE, bool DOWN, int MTR = 0, bool F16 = Cfg<TYPE, DOWN>::F16> struct Ops;
template <int TYPE, bool DOWN, int MTR> struct Ops<TYPE, DOWN, MTR, false> {
	using V = bf16x8;
	using F = Fac;
	__device__ static void factors(const BRegs<TYPE> &b, int st, int gi, F &f) { group_factors<TYPE, MTR>(b, st, gi, f); }
	__device__ static void deq(const BRegs<TYPE> &b, const F &f, const K16 &, int st, int s, V out[2])
	{
		deq_step<TYPE>(b, f, st, s, out);
	}
	__device__ static f32x16 mma(V a, V b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
};
template <int TYPE, bool DOWN, int MTR> struct Ops<TYPE, DOWN, MTR, true> {
	using V = f16x8;
	using F = typename std::conditional<TYPE == TIE_GGML_Q4_K, Fac16, Fac>::type;
	__device__ static void factors(const BRegs<TYPE> &b, int st, int gi, F &f)
	{
		if constexpr (TYPE == TIE_GGML_Q4_K)
			group_factors16<TYPE, MTR>(b, st, gi, f);
		else
			group_factors<TYPE, MTR>(b, st, gi, f);
	}
	template <bool NOD = false>
	__device__ static void deq(const BRegs<TYPE> &b, const F &f, const K16 &kc, int st, int s, V out[2])
	{
#if defined(TIE_DIAG_NODEQ)
		// diagnostic timing build: no dequantisation; one small f16 weight
		// per fragment (kept dependent on the loaded words, so their loads
		// stay) keeps the outputs finite and the epilogue on its usual path
		uint32_t w0, w1;
		if constexpr (TYPE == TIE_GGML_Q4_K) {
			w0 = b.q[0][0].x;
			w1 = b.q[1][0].x;
		} else {
			w0 = b.ql[0][0].x;
			w1 = b.ql[1][0].x;
		}
		const uint32_t h0 = 0x14001400u | (w0 & 0x00010001u), h1 = 0x14001400u | (w1 & 0x00010001u);
		out[0] = __builtin_bit_cast(V, u32x4{h0, h0, h0, h0});
		out[1] = __builtin_bit_cast(V, u32x4{h1, h1, h1, h1});
		return;
#endif
		if constexpr (TYPE == TIE_GGML_Q4_K)
			deq_step16<Cfg<TYPE, DOWN, MTR>::UH, NOD>(b, f, kc, s, out);
		else
			deq_step16_q6k<NOD>(b, f, kc, st, s, out);
	}
	__device__ static f32x16 mma(V a, V b, f32x16 c)
	{
#if defined(TIE_DIAG_NOMFMA)
		// diagnostic timing build: one VALU op in place of the MFMA
		c[0] += (float)a[0] * (float)b[0];
		return c;
#else
		return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
#endif
	}
};

// One stage of MFMAs over NMT live 32-row M tiles (BF16 weights, held in
// registers).  The A fragments of 16-K step s+1 are read from LDS while the
// MFMAs of step s run.
template <int TYPE, bool DOWN, int NMT, int MTR>
__device__ __forceinline__ void stage_mfma(const BRegs<TYPE> &b, int st, const uint8_t *__restrict__ A,
					   f32x16 acc[6][2])
{
	using C = Cfg<TYPE, DOWN, MTR>;
	constexpr int NA = NMT * C::NPL; // fragments per step (hi [+ lo] per tile)
	const int lane = threadIdx.x & 63;
	// fragment row r = 32 mt + lane%32 (swz(r) = swz(lane%32)), chunk 2s + lane/32
	const uint8_t *arow = A + (lane & 31) * C::RB;
	const int key = C::swz(lane & 31);
	auto read = [&](int s, bf16x8 fr[NA]) {
		const int slot = ((2 * s + (lane >> 5)) ^ key) * 16;
#pragma unroll
		for (int i = 0; i < NA; i++)
			fr[i] = *reinterpret_cast<const bf16x8 *>(arow + (i / NMT) * C::A_TILE + (i % NMT) * 32 * C::RB +
								  slot);
	};
	Fac f;
	group_factors<TYPE>(b, st, 0, f);
	bf16x8 fa[2][NA], fb[2][2];
	read(0, fa[0]);
	deq_step<TYPE>(b, f, st, 0, fb[0]);
#pragma unroll
	for (int s = 0; s < C::NSTEP; s++) {
		const int cur = s & 1;
#pragma unroll
		for (int i = 0; i < NA; i++) {
			const int mt = i % NMT;
			acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][0], acc[mt][0], 0, 0, 0);
			acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][1], acc[mt][1], 0, 0, 0);
		}
		if (s + 1 < C::NSTEP) {
			read(s + 1, fa[cur ^ 1]);
			if (TYPE == TIE_GGML_Q4_K && (s + 1) % 4 == 0)
				group_factors<TYPE>(b, st, (s + 1) / 4, f);
			deq_step<TYPE>(b, f, st, s + 1, fb[cur ^ 1]);
		}
		__builtin_amdgcn_sched_barrier(0);
	}
}

// ------------------------------------------------------------------ kernel
// One work tile with NMT live 32-row M tiles (nrows <= 32 NMT).
template <int TYPE, bool DOWN, int NMT, int MTR>
__device__ __forceinline__ void run_tile(const MfmaArgs &a, uint8_t *As, uint32_t *roff, int32_t *spair, int e,
					 int pbase, int nrows, int slab, int pair_id)
{
	using C = Cfg<TYPE, DOWN, MTR>;
	const int nk = a.in / C::KST;
	const int t = threadIdx.x;
#ifdef TIE_MFMA_TRACE
	const unsigned long long t_start = __builtin_readcyclecounter();
	unsigned long long t_loop = 0, bw_total = 0;
#endif
	const int w = __builtin_amdgcn_readfirstlane(t >> 6);
	const int lane = t & 63, h = lane >> 5;

	ASrc as;
	{
		const int rsub = lane / C::CPR, slot = lane % C::CPR;
		const int chunk = slot ^ C::swz(C::RPI * w + rsub);
		// Slot 2s + h of a stage holds the K of step s, lane half h.
		// Quantised weights: the 8-groups 1 and 2 of each 32-K quarter
		// swapped (lane half h takes code chunk h, a step half of it).
		// APERM: slots 0..3 are K 32p + ... of the half, slots 4..7 K 64 + 32p + ...
		const int q8 = C::SPLIT ? chunk & 3 : ((chunk & 1) << 1) | ((chunk >> 1) & 1);
		// UH: slot 2s + h holds the 8-group 4h + s (sub-block h, positions 8s ..)
		const int cofs = C::UH      ? 16 * (4 * (chunk & 1) + (chunk >> 1))
				 : C::APERM ? 128 * (chunk >> 2) + 16 * q8
					    : 64 * (chunk >> 2) + 16 * q8;
		as.base[0] = (const char *)a.a16;
		as.base[1] = (const char *)a.a16lo;
		as.cofs = cofs;
		// row r = RPI (NWAVES c + w') + rsub' is entry c of lane slot RPI w' + rsub'
		as.roff = roff + (C::RPI * w + rsub) * ROFF_STRIDE;
		as.nrows = nrows;
		if (t < C::MT) {
			const int r = t < nrows ? t : 0;
			const int pr = DOWN ? 0 : spair[r];
			const int row = DOWN ? pbase + r : pr / a.k;
			const int c = t / (C::RPI * NWAVES), ls = t % (C::RPI * NWAVES);
			roff[ls * ROFF_STRIDE + c] = (uint32_t)((size_t)row * a.in * 2);
		}
		__syncthreads();
	}
	BSrc bs;
#pragma unroll
	for (int j = 0; j < 2; j++) {
		const int mat = DOWN ? 0 : j;
		const int row = DOWN ? slab * DN_COLS + 64 * w + 32 * j + (lane & 31) : slab * GU_COLS + 32 * w + (lane & 31);
		const uint8_t *base = a.w[mat] + (size_t)e * a.expert_bytes[mat];
		if constexpr (TYPE == TIE_GGML_BF16)
			bs.p[j] = base + (size_t)row * a.in * 2;
		else
			bs.p[j] = base + (size_t)(row >> 6) * (a.in / QK) * panel_bytes(TYPE) + (row & 63) * 16;
		// d plane: 13 chunks after the panel start, 2 bytes per lane-row
		bs.dofs[j] = Q6K_CHUNKS * 1024 + 2 * (row & 63) - 16 * (row & 63);
	}

	f32x16 acc[6][2];
#pragma unroll
	for (int mt = 0; mt < NMT; mt++)
#pragma unroll
		for (int j = 0; j < 2; j++)
#pragma unroll
			for (int i = 0; i < 16; i++)
				acc[mt][j][i] = 0.0f;

	// the lane's two weight rows in the LDS panel buffer (quantised types)
	int bp[2], bi[2];
#pragma unroll
	for (int j = 0; j < 2; j++) {
		const int r = DOWN ? 64 * w + 32 * j + (lane & 31) : 32 * w + (lane & 31); // row within the matrix's tile
		bp[j] = DOWN ? r >> 6 : 2 * j + (r >> 6);
		bi[j] = r & 63;
	}
	uint8_t *Bs = As + C::LDS_A;

	if constexpr (C::B_LDS) {
		// Quantised weights, software-pipelined over the stages: a stage's
		// step s MFMAs run while the A fragments of step s+1 are read and its
		// weights dequantised; the next stage's DMA is issued after step 0's
		// MFMAs; the last step's MFMAs run after the stage barrier, while the
		// next stage's weights are read from LDS and its step 0 prepared.
		using O = Ops<TYPE, DOWN, MTR>;
		using V = typename O::V;
		constexpr int NA = NMT;
		static_assert(C::NPL == 1 && C::NSTEP % 2 == 0, "one activation plane, even step count");
		BDma<TYPE, MTR> bd;
		bdma_init<TYPE, DOWN, MTR>(a, e, slab, w, bd);
		constexpr int NS = C::NS;
		auto abuf = [&](int st) { return As + (st % NS) * C::ABUF; };
		auto bbuf = [&](int st) { return Bs + (st % NS) * C::BBUF; };
		// stage st's activations and weights into buffers st % NS
		auto issue = [&](int st) {
			if (st < nk) {
				dma_a<TYPE, DOWN, NMT, MTR>(as, st, w, abuf(st));
				dma_b<TYPE, DOWN, MTR>(bd, slab, st, w, bbuf(st));
			}
		};
		// direct loads one wave issues per stage (dma_a + dma_b)
		constexpr int NLIVE = (32 * NMT + NWAVES * C::RPI - 1) / (NWAVES * C::RPI);
		constexpr int PER = NLIVE * C::NPL + C::B_DMA;
		static_assert((NS - 2) * PER < 64, "vmcnt field");
		// end of stage st: stage st + 1's data landed (and this stage's LDS
		// reads done); the loads of the up to NS - 2 stages issued after it
		// may stay in flight (loads complete in order)
#ifdef TIE_MFMA_TRACE
		unsigned long long bwait = 0;
#endif
		auto barrier_after = [&](int st) {
#ifdef TIE_MFMA_TRACE
			const unsigned long long tb = __builtin_readcyclecounter();
#endif
			const int keep = min(NS - 2, nk - 2 - st);
			if (NS >= 4 && keep >= 2)
				stage_barrier_keep<(NS >= 4 ? 2 * PER : 0)>();
			else if (NS >= 3 && keep >= 1)
				stage_barrier_keep<(NS >= 3 ? PER : 0)>();
			else
				stage_barrier();
#ifdef TIE_MFMA_TRACE
			bwait += __builtin_readcyclecounter() - tb;
#endif
		};
		// fragment row r = 32 mt + lane%32 (swz(r) = swz(lane%32)), chunk 2s + lane/32
		const int arow = (lane & 31) * C::RB, key = C::swz(lane & 31);
		V fa[2][NA], fb[2][2];
		typename O::F f;
		BRegs<TYPE> b;
		const K16 kc = k16_consts();
		auto read = [&](int st, int s, V fr[NA]) {
			const uint8_t *A = abuf(st) + arow + ((2 * s + (lane >> 5)) ^ key) * 16;
#pragma unroll
			for (int i = 0; i < NA; i++)
				fr[i] = *reinterpret_cast<const V *>(A + i * 32 * C::RB);
		};
		// one-M-tile tiles: d applied per block (Q6_K: DF; Q4_K gate/up: QF,
		// with the minimum term from the sub-block sums)
		constexpr bool DF = TIE_MFMA_DFOLD && TYPE == TIE_GGML_Q6_K && NMT == 1 && MTR == MFMA_MT_TINY;
		constexpr bool QF = TIE_MFMA_QFOLD && C::UH && !DOWN && NMT == 1 && MTR == MFMA_MT_TINY;
		auto prep = [&](int st, int s, int slot) {
			read(st, s, fa[slot]);
			if (s == 0 || (TYPE == TIE_GGML_Q4_K && s % 4 == 0))
				O::factors(b, st, s / 4, f);
			O::template deq<DF || QF>(b, f, kc, st, s, fb[slot]);
		};
		auto mm = [&](int slot) {
#pragma unroll
			for (int i = 0; i < NA; i++) {
				acc[i][0] = O::mma(fa[slot][i], fb[slot][0], acc[i][0]);
				acc[i][1] = O::mma(fa[slot][i], fb[slot][1], acc[i][1]);
			}
		};
		constexpr int L = (C::NSTEP - 1) & 1; // slot of a stage's last step
		// all steps but the last of stage st (the DMA of stage st + NS - 1
		// with more)
		auto steps = [&](int st, bool more) {
#pragma unroll
			for (int s = 0; s + 1 < C::NSTEP; s++) {
				mm(s & 1);
				// the buffers written here were last read in stage st - 1,
				// which every wave has left (its barrier)
				if (s == 0 && more)
					issue(st + NS - 1);
				prep(st, s + 1, (s & 1) ^ 1);
				__builtin_amdgcn_sched_barrier(0);
			}
		};
#pragma unroll
		for (int i = 0; i + 1 < NS; i++)
			issue(i);
		barrier_after(-1);
		if constexpr (DF || QF) {
			// as below, block by block: the block's MFMAs into accb (from
			// zero), then acc += d 2^S accb per lane column (fp32).  QF: and
			// acc += S M, the block's 8 sub-block sums of the row's A (high
			// parts in lane half 0, remainders in half 1) times the column's
			// 8 minimum factors (in both halves)
			static_assert(C::SPB * C::KST == QK, "stages per block");
			f32x16 accb[2];
			const uint16_t *xs = nullptr;
			V sa;
			if constexpr (QF) {
				const int r = lane & 31;
				const int tok = spair[r < nrows ? r : 0] / a.k;
				xs = a.xsum + (size_t)(2 * tok + h) * (a.in / 32);
				sa = *reinterpret_cast<const V *>(xs);
			}
			for (int st0 = 0; st0 < nk; st0 += C::SPB) {
#pragma unroll
				for (int sb = 0; sb < C::SPB; sb++) {
					const int st = st0 + sb;
					issue(st + NS - 1);
					lds_b<TYPE, MTR>(bbuf(st), bp, bi, st, h, b);
					prep(st, 0, 0);
#pragma unroll
					for (int s = 0; s < C::NSTEP; s++) {
#pragma unroll
						for (int j = 0; j < 2; j++)
							accb[j] = O::mma(fa[s & 1][0], fb[s & 1][j],
									 (sb == 0 && s == 0) ? f32x16{} : accb[j]);
						if (s + 1 < C::NSTEP)
							prep(st, s + 1, (s & 1) ^ 1);
						__builtin_amdgcn_sched_barrier(0);
					}
					if (sb + 1 == C::SPB) {
#pragma unroll
						for (int j = 0; j < 2; j++) {
							float D;
							if constexpr (QF)
								D = (float)f.DM[j][0][0]; // d 2^S (exact in f16)
							else
								D = f.d6[j] * (float)(1 << F16_SHIFT);
#pragma unroll
							for (int i = 0; i < 16; i++)
								acc[0][j][i] = __builtin_fmaf(D, accb[j][i], acc[0][j][i]);
							if constexpr (QF)
								acc[0][j] = O::mma(sa, q4k_mins16(b.sc[j]), acc[0][j]);
						}
						if constexpr (QF) {
							if (st0 + C::SPB < nk)
								sa = *reinterpret_cast<const V *>(xs + 8 * ((st0 + C::SPB) / C::SPB));
						}
					}
					barrier_after(st);
				}
			}
		} else if constexpr (NMT < TIE_MFMA_PIPE_NMT) {
			// few MFMAs per step: each stage self-contained (the DMA of stage
			// st + NS - 1 first, then its weights from LDS, then the steps)
			for (int st = 0; st < nk; st++) {
				issue(st + NS - 1);
				lds_b<TYPE, MTR>(bbuf(st), bp, bi, st, h, b);
				prep(st, 0, 0);
#pragma unroll
				for (int s = 0; s < C::NSTEP; s++) {
					mm(s & 1);
					if (s + 1 < C::NSTEP)
						prep(st, s + 1, (s & 1) ^ 1);
					__builtin_amdgcn_sched_barrier(0);
				}
				barrier_after(st);
			}
		} else {
			lds_b<TYPE>(bbuf(0), bp, bi, 0, h, b);
			prep(0, 0, 0);
			for (int st = 0; st + 1 < nk; st++) {
				steps(st, true);
				// the last step's fragments are in registers: the barrier only
				// waits for stage st + 1's data and this stage's LDS reads
				barrier_after(st);
				lds_b<TYPE>(bbuf(st + 1), bp, bi, st + 1, h, b);
				mm(L);
				prep(st + 1, 0, L ^ 1);
				// order: the LDS reads, two MFMAs (their latency), then the
				// preparation's VALU work spread between the other MFMAs
				__builtin_amdgcn_sched_group_barrier(0x100, 32, 0);
				__builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
#pragma unroll
				for (int i = 2; i < 2 * NA; i++) {
					__builtin_amdgcn_sched_group_barrier(0x002, TIE_MFMA_TAIL_VALU, 0);
					__builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
				}
				__builtin_amdgcn_sched_barrier(0);
			}
			steps(nk - 1, false);
			stage_barrier(); // every wave's LDS reads done before the epilogue reuses the buffers
			mm(L);
		}
#ifdef TIE_MFMA_TRACE
		bw_total = bwait;
#endif
	} else if constexpr (TIE_BF16_B3) {
		// weights two stages ahead: the loads of stage st + 2 (issued last,
		// 8 vector loads per lane) stay in flight across the stage barrier,
		// so each stage's weights have two stages of MFMAs to arrive in
		BRegs<TYPE> b0, b1, b2;
		load_b<TYPE>(bs, 0, h, b0);
		dma_a<TYPE, DOWN, NMT, MTR>(as, 0, w, As);
		if (nk > 1) {
			load_b<TYPE>(bs, 1, h, b1);
			stage_barrier_keep<8>();
		} else {
			stage_barrier();
		}
		auto body = [&](int st, BRegs<TYPE> &cur, BRegs<TYPE> &n2) {
			if (st + 1 < nk)
				dma_a<TYPE, DOWN, NMT, MTR>(as, st + 1, w, As + ((st + 1) & 1) * C::ABUF);
			if (st + 2 < nk)
				load_b<TYPE>(bs, st + 2, h, n2);
			stage_mfma<TYPE, DOWN, NMT, MTR>(cur, st, As + (st & 1) * C::ABUF, acc);
			if (st + 2 < nk)
				stage_barrier_keep<8>();
			else
				stage_barrier();
		};
		for (int st = 0; st < nk; st += 3) {
			body(st, b0, b2);
			if (st + 1 < nk)
				body(st + 1, b1, b0);
			if (st + 2 < nk)
				body(st + 2, b2, b1);
		}
	} else {
		BRegs<TYPE> b0, b1;
		load_b<TYPE>(bs, 0, h, b0);
		dma_a<TYPE, DOWN, NMT, MTR>(as, 0, w, As);
		stage_barrier();

		// stage st: the weights (registers) and activations (the other LDS
		// buffer) of st+1 are fetched, then the MFMAs of st run
		auto body = [&](int st, BRegs<TYPE> &cur, BRegs<TYPE> &nxt) {
			if (st + 1 < nk) {
				load_b<TYPE>(bs, st + 1, h, nxt);
				dma_a<TYPE, DOWN, NMT, MTR>(as, st + 1, w, As + ((st + 1) & 1) * C::ABUF);
			}
			stage_mfma<TYPE, DOWN, NMT, MTR>(cur, st, As + (st & 1) * C::ABUF, acc);
			stage_barrier();
		};
		for (int st = 0; st < nk; st += 2) {
			body(st, b0, b1);
			if (st + 1 < nk)
				body(st + 1, b1, b0);
		}
	}

#ifdef TIE_MFMA_TRACE
	t_loop = __builtin_readcyclecounter();
#endif
	if constexpr (DOWN) {
		// the tile's pair ids, for the epilogue's y rows and token flags (the
		// down kernel's activation rows are the tile's dense h rows, so its
		// stages never waited for these: loaded in the prologue, in a
		// register until now)
		if (t < nrows)
			spair[t] = pair_id;
		__syncthreads();
	}
	// gate/up: TIE's SiLU table (32 KiB) into the now idle stage buffers, so
	// the epilogue's table lookups are LDS reads
	const float *silu = a.silu;
	if constexpr (C::SILU_LDS) {
		static_assert(SILU_N * 4 <= C::STAGE_BYTES, "SiLU table must fit the stage buffers");
#pragma unroll
		for (int c = 0; c < SILU_N * 4 / 1024 / NWAVES; c++) {
			const int off = 1024 * (NWAVES * c + w);
			dma16(reinterpret_cast<const uint8_t *>(a.silu) + off + 16 * lane,
			      __builtin_amdgcn_readfirstlane(lds_addr(As + off)));
		}
		stage_barrier();
		silu = reinterpret_cast<const float *>(As);
	}
	// D layout of v_mfma_f32_32x32x16: lane l, register i holds
	// row 8*(i/4) + 4*(l/32) + i%4, column l%32.
	if constexpr (C::F16 && !C::SPLIT) {
		// 16-bit outputs of the f16 kernels through a wave-private LDS tile
		// (fp32, rows padded so the two row groups of a write fall in
		// different banks), then 16-byte coalesced stores: gate/up h rows
		// (32 columns of the wave) at 32 KiB past the SiLU table, down y
		// rows (64 columns) at the buffers' start.
		constexpr int NC = DOWN ? 64 : 32;          // columns of the wave
		constexpr int LS = DOWN ? 72 : 40;          // LDS row stride (floats)
		// half an M tile (16 rows) at a time: registers i = 8 half .. 8 half + 7
		// hold rows 16 half .. 16 half + 15
		float *tl = reinterpret_cast<float *>(As + (C::SILU_LDS ? 32768 : 0) + w * (16 * LS * 4));
		static_assert((C::SILU_LDS ? 32768 : 0) + NWAVES * 16 * LS * 4 <= C::STAGE_BYTES, "epilogue tile");
		const int c0 = lane & 31;
		// gate/up: K positions 1, 2 (and 5, 6) of each 8-group of h swapped
		// (the dequantised pairs' order)
		const int pc0 = DOWN ? c0 : (c0 & ~3) | ((c0 & 1) << 1) | ((c0 >> 1) & 1);
#pragma unroll
		for (int mt = 0; mt < NMT; mt++) {
#pragma unroll
			for (int half = 0; half < 2; half++) {
				// (a half without rows of the tile has nothing to store; the
				// 32- and 64-row tile kernels: 30B T=32 -1.3%, T=22 -2.2%,
				// LFM2 T=32 -1.4%; the large tiles, mostly full, measured
				// no gain)
				if (TIE_MFMA_EPI_SKIP && MTR != 0 && 32 * mt + 16 * half >= nrows)
					continue;
				if constexpr (DOWN) {
#pragma unroll
					for (int ii = 0; ii < 8; ii++) {
						const int i = 8 * half + ii;
						const int r = 8 * (ii >> 2) + 4 * h + (ii & 3); // row within the half
						tl[r * LS + c0] = acc[mt][0][i] * a.y_scale;
						tl[r * LS + 32 + c0] = acc[mt][1][i] * a.y_scale;
					}
				} else {
					// TIE's table SwiGLU (tie_swiglu, the same operations) on
					// the half's 8 values, all table reads issued together
					constexpr float unscale = 1.0f / (1 << F16_SHIFT);
					float pos[8], up[8], y1[8], y2[8];
					int idx[8];
#pragma unroll
					for (int ii = 0; ii < 8; ii++) {
						const int i = 8 * half + ii;
						const float g = acc[mt][0][i] * unscale;
						up[ii] = acc[mt][1][i] * unscale;
						pos[ii] = ((g + 10.0f) * 8191.0f) * 0.05f;
						int id = (pos[ii] >= -2147483648.0f && pos[ii] < 2147483648.0f)
								 ? (int)__builtin_rintf(pos[ii])
								 : (int)0x80000000;
						id = id < 0 ? 0 : id;
						idx[ii] = id > SILU_N - 2 ? SILU_N - 2 : id;
					}
#pragma unroll
					for (int ii = 0; ii < 8; ii++) {
						y1[ii] = silu[idx[ii]];
						y2[ii] = silu[idx[ii] + 1];
					}
					uint32_t bad = 0;
#pragma unroll
					for (int ii = 0; ii < 8; ii++) {
						const int r = 8 * (ii >> 2) + 4 * h + (ii & 3); // row within the half
						const float frac = pos[ii] - (float)idx[ii];
						const float sl = __builtin_fmaf(frac, y2[ii] - y1[ii], y1[ii]);
						const float hs = (sl * up[ii]) * a.h_scale;
						tl[r * LS + pc0] = hs;
						const int mrow = 32 * mt + 16 * half + r;
						bad |= (!(__builtin_fabsf(hs) < 65504.0f) && mrow < nrows) ? 1u << ii : 0u;
					}
					// a value outside the f16 range sends the pair's token to
					// the exact recomputation (rare: off the common path)
					if (bad) {
						for (int ii = 0; ii < 8; ii++)
							if (bad & (1u << ii)) {
								const int r = 8 * (ii >> 2) + 4 * h + (ii & 3);
								const int tok = spair[32 * mt + 16 * half + r] / a.k;
								if (a.tok_flag[tok] == 0) // listed already: no atomic
									flag_token(a.tok_flag, a.fix_list, a.fix_count, tok);
							}
					}
				}
				__builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): the tile's LDS writes done
				__builtin_amdgcn_wave_barrier();
				// 16-byte chunks: 16 rows x NC columns / 8 per chunk, 64 lanes
				constexpr int CPRW = NC / 8; // chunks per row
#pragma unroll
				for (int q = 0; q < 16 * CPRW / 64; q++) {
					const int cidx = lane + 64 * q, r = cidx / CPRW, part = cidx % CPRW;
					// down: odd rows read their second 4 columns first, so
					// the two rows of a 16-lane read group fall in different
					// banks (row stride 72 floats: 8 banks apart)
					const int sw = DOWN ? 4 * (r & 1) : 0;
					float4 u0 = *reinterpret_cast<const float4 *>(tl + r * LS + 8 * part + sw);
					float4 u1 = *reinterpret_cast<const float4 *>(tl + r * LS + 8 * part + 4 - sw);
					// (kept as two reads at these addresses, not folded into
					// reads of the selected addresses)
					asm volatile("" : "+v"(u0.x), "+v"(u0.y), "+v"(u0.z), "+v"(u0.w), "+v"(u1.x), "+v"(u1.y),
						     "+v"(u1.z), "+v"(u1.w));
					const float4 v0 = sw ? u1 : u0, v1 = sw ? u0 : u1;
					const int mrow = 32 * mt + 16 * half + r;
					if (mrow < nrows) {
						if (DOWN && a.y16) {
							// experts: y [pair][d] as f16(y 2^-y_shift); a value
							// outside the f16 range sends the pair's token to
							// the exact recomputation
							const f16x8 yv = {(_Float16)v0.x, (_Float16)v0.y, (_Float16)v0.z, (_Float16)v0.w,
									  (_Float16)v1.x, (_Float16)v1.y, (_Float16)v1.z, (_Float16)v1.w};
							uint16_t *yr = a.y16 + (size_t)spair[mrow] * a.rows + slab * DN_COLS + 64 * w + 8 * part;
							*reinterpret_cast<f16x8 *>(yr) = yv;
							const float m = __builtin_fmaxf(
								__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v0.x), __builtin_fabsf(v0.y)),
										__builtin_fmaxf(__builtin_fabsf(v0.z), __builtin_fabsf(v0.w))),
								__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v1.x), __builtin_fabsf(v1.y)),
										__builtin_fmaxf(__builtin_fabsf(v1.z), __builtin_fabsf(v1.w))));
							// fmax drops NaN: the sum of the eight is NaN if any is
							const bool nan = (v0.x + v0.y + v0.z + v0.w + v1.x + v1.y + v1.z + v1.w) !=
									 (v0.x + v0.y + v0.z + v0.w + v1.x + v1.y + v1.z + v1.w);
							if (nan || !(m < 65504.0f)) {
								const int tok = spair[mrow] / a.k;
								if (a.tok_flag[tok] == 0) // listed already: no atomic
									flag_token(a.tok_flag, a.fix_list, a.fix_count, tok);
							}
						} else if (DOWN) {
							// fp32 rows: out [token][rows] (dense matrices)
							float *orow = a.y + (size_t)spair[mrow] * a.rows + slab * DN_COLS + 64 * w + 8 * part;
							*reinterpret_cast<float4 *>(orow) = v0;
							*reinterpret_cast<float4 *>(orow + 4) = v1;
						} else {
							const f16x8 hv = {(_Float16)v0.x, (_Float16)v0.y, (_Float16)v0.z, (_Float16)v0.w,
									  (_Float16)v1.x, (_Float16)v1.y, (_Float16)v1.z, (_Float16)v1.w};
							uint16_t *hr =
								a.h16 + (size_t)(pbase + mrow) * a.rows + slab * GU_COLS + 32 * w + 8 * part;
							*reinterpret_cast<f16x8 *>(hr) = hv;
						}
					}
				}
				__builtin_amdgcn_s_waitcnt(0xc07f);
				__builtin_amdgcn_wave_barrier(); // the reads done before the next half overwrites
			}
			__builtin_amdgcn_sched_barrier(0);
		}
	} else
#pragma unroll
	for (int mt = 0; mt < NMT; mt++) {
#pragma unroll
		for (int i = 0; i < 16; i++) {
			const int mrow = 32 * mt + 8 * (i >> 2) + 4 * h + (i & 3);
			if (mrow >= nrows)
				continue;
			const int p = pbase + mrow;
			if (!DOWN) {
				const int col = slab * GU_COLS + 32 * w + (lane & 31);
				constexpr float unscale = C::F16 ? 1.0f / (1 << F16_SHIFT) : 1.0f;
				const float hv = tie_swiglu(acc[mt][0][i] * unscale, acc[mt][1][i] * unscale, silu);
				if (a.h_f16) {
					// f16, K positions 1, 2 (and 5, 6) of each 8-group swapped
					// (the dequantised pairs' order).  A value outside the f16
					// range sends the pair's token to the exact recomputation.
					const int pc = (col & ~3) | ((col & 1) << 1) | ((col >> 1) & 1);
					const float hs = hv * a.h_scale;
					a.h16[(size_t)p * a.rows + pc] = __builtin_bit_cast(uint16_t, (_Float16)hs);
					if (!(__builtin_fabsf(hs) < 65504.0f)) {
						const int tok = spair[mrow] / a.k;
						if (a.tok_flag[tok] == 0) // listed already: no atomic
							flag_token(a.tok_flag, a.fix_list, a.fix_count, tok);
					}
				} else {
					const uint16_t hi = bf16_bits(hv);
					a.h16[(size_t)p * a.rows + col] = hi;
					if (C::SPLIT)
						a.h16lo[(size_t)p * a.rows + col] = bf16_bits(hv - bf16_bits_to_float(hi));
				}
			} else {
				// y in fp32; the f16 weights' factor 2^F16_SHIFT and h's
				// scale come out here (a power of two: exact)
				const float unscale = C::F16 ? a.y_scale : 1.0f;
				float *yr = a.y + (size_t)spair[mrow] * a.rows + slab * DN_COLS + 64 * w + (lane & 31);
				yr[0] = acc[mt][0][i] * unscale;
				yr[32] = acc[mt][1][i] * unscale;
			}
		}
		// one M tile at a time: only its accumulators move to VGPRs
		__builtin_amdgcn_sched_barrier(0);
	}
#ifdef TIE_MFMA_TRACE
	if (t == 0 && t_loop) {
		const unsigned long long t_end = __builtin_readcyclecounter();
		atomicAdd(&g_mfma_trace[DOWN][0], t_end - t_start);
		atomicAdd(&g_mfma_trace[DOWN][1], bw_total);
		atomicAdd(&g_mfma_trace[DOWN][2], t_end - t_loop);
		atomicAdd(&g_mfma_trace[DOWN][3], 1ull);
	}
#endif
}

// waves per SIMD: the quantised kernels keep their LDS and registers small
// enough for two workgroups per CU; the BF16 kernels (weights prefetched
// into registers) run one wave per SIMD
constexpr int mf_wpe(int type, bool down, int mtr)
{
	return type == TIE_GGML_BF16 ? (down ? TIE_MFMA_BF16_DN_WPE : TIE_MFMA_BF16_WPE)
	       : mtr == MFMA_MT_TINY ? (down ? TIE_MFMA_TINY_DN_WPC : TIE_MFMA_TINY_GU_WPC)
	       : mtr && !down ? 3 : down ? TIE_MFMA_DN_WPE : TIE_MFMA_GU_WPE;
}

template <int TYPE, bool DOWN, int MTR>
__global__ __launch_bounds__(MF_THREADS) __attribute__((amdgpu_waves_per_eu(mf_wpe(TYPE, DOWN, MTR), mf_wpe(TYPE, DOWN, MTR)))) void
mfma_experts_kernel(MfmaArgs a)
{
	using C = Cfg<TYPE, DOWN, MTR>;
	constexpr int MT = C::MT, MT_TILES = C::MT / 32;
	extern __shared__ __attribute__((aligned(16))) uint8_t As[]; // A [2][ABUF] | B [2][BBUF] | row offsets
	uint32_t *roff = reinterpret_cast<uint32_t *>(As + C::STAGE_BYTES);
	int32_t *spair = reinterpret_cast<int32_t *>(roff + C::RPI * NWAVES * ROFF_STRIDE);

	// The work tiles: expert e's pairs (a.cnt[e] of them, bucket e) split
	// evenly over ceil(cnt / MT) tiles, the tiles numbered in expert order.
	// Every workgroup derives its tile from the counts: exclusive scans of
	// the tile and pair counts over the experts (thread i owns experts
	// 4i .. 4i + 3), in the idle stage buffers.
#ifdef TIE_MFMA_TRACE
	const unsigned long long t_k0 = __builtin_readcyclecounter();
#endif
#ifdef TIE_MFMA_TIMELINE
	const unsigned long long tl0 = __builtin_amdgcn_s_memrealtime();
#endif
	int e, slab, pbase, nrows, pair_id = 0;
	if (MTR == MFMA_MT_TINY && a.direct) {
		// one item per (expert, column slab), mapped to the workgroups in the
		// same XCD-aware order as the tile list's items (the slabs of an
		// expert on one XCD); the expert's count and its pair ids (at most
		// MFMA_DIRECT_T, read before the count is known) in one memory round
		// trip
		const int nslab = gridDim.x;
		const int live = a.E * nslab;
		const int per_xcd = (live + 7) / 8;
		const int lin = blockIdx.y * gridDim.x + blockIdx.x;
		const int v = (lin % 8) * per_xcd + lin / 8;
		if (lin / 8 >= per_xcd || v >= live)
			return;
		e = v / nslab;
		slab = v % nslab;
		const int t = threadIdx.x;
		if (t < MFMA_DIRECT_T && t < a.bstride)
			pair_id = a.bucket[(size_t)e * a.bstride + t];
		nrows = a.cnt[e];
		if (nrows == 0)
			return;
		pbase = e * MFMA_DIRECT_T;
	} else {
		const int mtc = a.mt_cap > 0 && a.mt_cap < MT ? a.mt_cap : MT;
		int li, off;
		{
			int *sc = reinterpret_cast<int *>(As); // [2 MF_THREADS / 64] scan | e, li, off
			const int t = threadIdx.x;
			int c4[4], n4[4], csum = 0, nsum = 0;
#pragma unroll
			for (int i = 0; i < 4; i++) {
				const int ex = 4 * t + i;
				c4[i] = ex < a.E ? a.cnt[ex] : 0;
				n4[i] = (c4[i] + mtc - 1) / mtc;
				csum += c4[i];
				nsum += n4[i];
			}
			// one scan of both sums (tiles in the high word, pairs in the low)
			long long tot;
			const long long b2 = block_exclusive_scan64<MF_THREADS>(((long long)nsum << 32) | (long long)csum,
										 reinterpret_cast<long long *>(sc), tot);
			const int ntiles = (int)(tot >> 32);
			int nbase = (int)(b2 >> 32), cbase = (int)(b2 & 0xffffffffll);
			// this workgroup's item (XCD-aware order: consecutive workgroup ids
			// go round-robin over the 8 XCDs, each with its own L2; the id is
			// remapped so that each XCD takes a contiguous run of (tile, column
			// slab) items, and the slabs of one expert tile share an XCD and read
			// the tile's gathered activation rows from its L2)
			const int nslab = gridDim.x;
			const int live = ntiles * nslab;
			const int per_xcd = (live + 7) / 8;
			const int lin = blockIdx.y * gridDim.x + blockIdx.x;
			const int v = (lin % 8) * per_xcd + lin / 8;
			if (lin / 8 >= per_xcd || v >= live)
				return;
			const int tile = v / nslab;
			slab = v % nslab;
#pragma unroll
			for (int i = 0; i < 4; i++) {
				if (tile >= nbase && tile < nbase + n4[i]) {
					sc[2 * MF_THREADS / 64] = 4 * t + i;
					sc[2 * MF_THREADS / 64 + 1] = tile - nbase;
					sc[2 * MF_THREADS / 64 + 2] = cbase;
				}
				nbase += n4[i];
				cbase += c4[i];
			}
			__syncthreads();
			e = sc[2 * MF_THREADS / 64];
			li = sc[2 * MF_THREADS / 64 + 1];
			off = sc[2 * MF_THREADS / 64 + 2];
			__syncthreads(); // the stage buffers are free again
		}
		const int cnt = a.cnt[e];
		const int ntl = (cnt + mtc - 1) / mtc;
		const int rpt = (cnt + ntl - 1) / ntl;
		const int m0 = li * rpt;
		pbase = off + m0; // the tile's first row in the dense h rows
		nrows = min(rpt, cnt - m0);
		// the tile's pair ids (rows m0 .. m0 + nrows - 1 of the expert's bucket):
		// gate/up gathers its activation rows by them, the down kernel needs
		// them only in its epilogue (run_tile stores them there)
		if (threadIdx.x < nrows)
			pair_id = a.bucket[(size_t)e * a.bstride + m0 + threadIdx.x];
	}
	if constexpr (!DOWN) {
		if (threadIdx.x < nrows)
			spair[threadIdx.x] = pair_id;
		__syncthreads();
	}
#ifdef TIE_MFMA_TRACE
	if (threadIdx.x == 0)
		atomicAdd(&g_mfma_trace[DOWN][4], __builtin_readcyclecounter() - t_k0);
#endif
#ifdef TIE_MFMA_FIXED_NMT
	// one tile height for every tile (one copy of run_tile's code)
	run_tile<TYPE, DOWN, MT_TILES, MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
	return;
#endif
	switch ((nrows + 31) >> 5) {
	case 1:
		run_tile<TYPE, DOWN, 1, MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
		break;
	case 2:
		if constexpr (MT_TILES >= 2)
			run_tile<TYPE, DOWN, (MT_TILES >= 2 ? 2 : 1), MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
		break;
	case 3:
		if constexpr (MT_TILES >= 3)
			run_tile<TYPE, DOWN, (MT_TILES >= 3 ? 3 : 1), MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
		break;
	case 4:
		if constexpr (MT_TILES >= 4)
			run_tile<TYPE, DOWN, (MT_TILES >= 4 ? 4 : 1), MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
		break;
	case 5:
		if constexpr (MT_TILES >= 5)
			run_tile<TYPE, DOWN, (MT_TILES >= 5 ? 5 : 1), MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
		break;
	default:
		if constexpr (MT_TILES >= 6)
			run_tile<TYPE, DOWN, (MT_TILES >= 6 ? 6 : 1), MTR>(a, As, roff, spair, e, pbase, nrows, slab, pair_id);
	}
#ifdef TIE_MFMA_TIMELINE
	{
		const int lin = blockIdx.y * gridDim.x + blockIdx.x;
		if (threadIdx.x == 0 && lin < MFMA_TL_WG) {
			g_mfma_tl[DOWN][lin][0] = tl0;
			g_mfma_tl[DOWN][lin][1] = __builtin_amdgcn_s_memrealtime();
		}
	}
#endif
}

// ------------------------------------------------------------ routing
// The matrix-core path's selection and grouping, one wave per token, after
// the router logits: top-k + softmax (topk_softmax: find_top_k and softmax,
// engine.c:864-914), then each selected expert e records the slot that
// chose it, sel[e][t] = j + 1 (a byte of its own: no atomics; the array is
// zeroed by the logits kernel).  bucket_plan_kernel turns these rows into
// per-expert pair lists.  Up to ROUTE_APPEND_MAX_T tokens the wave appends
// its pairs to the lists itself instead (one atomic on the expert's count,
// zeroed by the logits kernel, per pair; few pairs per count at these
// sizes), and bucket_plan does not run: the order of pairs in a list then
// varies from call to call, which changes no result (each pair's rows are
// computed on their own, and h and y are addressed through the list or by
// pair id).  The same wave converts the token's x row into the
// gate/up A operand:
//   MODE 0: bf16
//   MODE 1: f16 with the K order inside each 8-group 0,2,1,3,4,6,5,7 (the
//           order of the dequantised weight pairs); the token is flagged
//           and listed for the exact recomputation when any x is not finite
//           or not below 65504 in magnitude
//   MODE 2: bf16 high and remainder planes (BF16 weights)
constexpr int RB_THREADS = 256;
struct BucketArgs {
	const float *logits;
	int T, ts, E, k, d, routing; // ts: row stride of sel (T rounded up to 4)
	const float *pbias;
	int32_t *topk_idx;
	float *topk_w;
	uint8_t *sel;
	int32_t *cnt, *bucket; // non-null: append the pairs to the lists directly (small T)
	int converted;         // MODE 1: the logits kernel wrote the A operand and flag[t] already
	const float *x;
	uint16_t *xa, *xlo;
	int32_t *flag, *list, *count;
	uint16_t *xsum; // MODE 1, non-null: also the sub-block sums of the A operand (Workspace::xsum)
};

// Sub-block sums of one token's f16 A row (MODE 1): lane group 4m..4m+3
// holds the 8-groups of one 32-K sub-block (its lanes' 8-value sums in
// fp32, then two lane exchanges); the first lane stores the f16 high and
// remainder parts.  A sum outside the f16 range flags the token.
__device__ __forceinline__ int store_xsum(uint16_t *xs, int t, int nsub, int sb, float part, bool store)
{
	part += __shfl_xor(part, 1);
	part += __shfl_xor(part, 2);
	if (!store || (threadIdx.x & 3) != 0)
		return 0;
	const _Float16 hi = (_Float16)part;
	const _Float16 lo = (_Float16)(part - (float)hi);
	xs[(size_t)(2 * t) * nsub + sb] = __builtin_bit_cast(uint16_t, hi);
	xs[(size_t)(2 * t + 1) * nsub + sb] = __builtin_bit_cast(uint16_t, lo);
	return !(__builtin_fabsf(part) < 65504.0f);
}

template <int MODE> __global__ __launch_bounds__(RB_THREADS) void route_bucket_kernel(BucketArgs r)
{
	__shared__ uint64_t etab[32];
	if (threadIdx.x < 32) {
		const uint64_t tab[32] = TIE_EXP2_TABLE;
		etab[threadIdx.x] = tab[threadIdx.x];
	}
	__syncthreads();
	const int lane = threadIdx.x & 63;
	const int t = blockIdx.x * (RB_THREADS / 64) + (threadIdx.x >> 6);
	if (t >= r.T)
		return;
	// the token's x row in flight during the selection: RB_X float4 per
	// lane per round (8 consecutive floats, one f16x8 of the A row, per
	// pair of float4)
	constexpr int RB_X = 8;
	const float4 *xr = reinterpret_cast<const float4 *>(r.x + (size_t)t * r.d);
	const int n4 = r.d / 4;
	float4 xv[RB_X];
	const bool conv = !(MODE == 1 && r.converted);
	if (conv) {
#pragma unroll
		for (int i = 0; i < RB_X / 2; i++) {
			const int q = 2 * (lane + 64 * i);
			xv[2 * i] = q < n4 ? xr[q] : make_float4(0, 0, 0, 0);
			xv[2 * i + 1] = q < n4 ? xr[q + 1] : make_float4(0, 0, 0, 0);
		}
	}
	topk_softmax(r.logits + (size_t)t * r.E, r.E, r.k, etab, r.topk_idx + (size_t)t * r.k, r.topk_w + (size_t)t * r.k,
		     r.routing, r.pbias);
	if (lane < r.k) {
		// lane j wrote slot j above
		const int e = r.topk_idx[(size_t)t * r.k + lane];
		if (e >= 0) {
			if (r.cnt)
				r.bucket[(size_t)e * r.ts + atomicAdd(r.cnt + e, 1)] = t * r.k + lane;
			else
				r.sel[(size_t)e * r.ts + t] = (uint8_t)(lane + 1);
		}
	}
	if constexpr (MODE == 1) {
		if (!conv) {
			// the A operand and the flag came with the logits: its sub-block
			// sums from it, then list the token
			int sbad = 0;
			if (r.xsum) {
				const int nsub = r.d / 32;
				const f16x8 *xr8 = reinterpret_cast<const f16x8 *>(r.xa + (size_t)t * r.d);
				for (int g0 = 0; g0 < r.d / 8; g0 += 64) {
					const int g8 = g0 + lane;
					float part = 0.0f;
					if (g8 < r.d / 8) {
						const f16x8 v = xr8[g8];
#pragma unroll
						for (int i = 0; i < 8; i++)
							part += (float)v[i];
					}
					sbad |= store_xsum(r.xsum, t, nsub, g8 >> 2, part, g8 < r.d / 8);
				}
				sbad = __any(sbad);
			}
			if (lane == 0 && sbad && !r.flag[t])
				r.flag[t] = 1;
			if (lane == 0 && r.flag[t])
				r.list[atomicAdd(r.count, 1)] = t;
			return;
		}
	}
	int bad = 0;
	for (int base = 0; base < n4; base += 128 * (RB_X / 2)) {
		if (base > 0) {
#pragma unroll
			for (int i = 0; i < RB_X / 2; i++) {
				const int q = base + 2 * (lane + 64 * i);
				xv[2 * i] = q < n4 ? xr[q] : make_float4(0, 0, 0, 0);
				xv[2 * i + 1] = q < n4 ? xr[q + 1] : make_float4(0, 0, 0, 0);
			}
		}
#pragma unroll
		for (int i = 0; i < RB_X / 2; i++) {
			const int q = base + 2 * (lane + 64 * i); // float4 index of the pair's first half
			if constexpr (MODE == 1) {
				// sub-block sums of the f16 values (every lane takes part in
				// the exchanges)
				if (r.xsum) {
					float part = 0.0f;
					if (q < n4) {
						const float4 a = xv[2 * i], c = xv[2 * i + 1];
						part = (((((((float)(_Float16)a.x + (float)(_Float16)a.y) + (float)(_Float16)a.z) +
							   (float)(_Float16)a.w) + (float)(_Float16)c.x) + (float)(_Float16)c.y) +
							 (float)(_Float16)c.z) + (float)(_Float16)c.w;
					}
					bad |= store_xsum(r.xsum, t, r.d / 32, (q / 2) >> 2, part, q < n4);
				}
			}
			if (q >= n4)
				continue;
			const float4 a = xv[2 * i], c = xv[2 * i + 1];
			if constexpr (MODE == 1) {
				const float m = __builtin_fmaxf(
					__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(a.x), __builtin_fabsf(a.y)),
							__builtin_fmaxf(__builtin_fabsf(a.z), __builtin_fabsf(a.w))),
					__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(c.x), __builtin_fabsf(c.y)),
							__builtin_fmaxf(__builtin_fabsf(c.z), __builtin_fabsf(c.w))));
				// fmax drops NaN: test the values themselves for NaN
				const bool nan = a.x != a.x || a.y != a.y || a.z != a.z || a.w != a.w || c.x != c.x ||
						 c.y != c.y || c.z != c.z || c.w != c.w;
				bad |= (nan || !(m < 65504.0f)) ? 1 : 0;
				const f16x8 h = {(_Float16)a.x, (_Float16)a.z, (_Float16)a.y, (_Float16)a.w,
						 (_Float16)c.x, (_Float16)c.z, (_Float16)c.y, (_Float16)c.w};
				reinterpret_cast<f16x8 *>(r.xa + (size_t)t * r.d)[q / 2] = h;
			} else if constexpr (MODE == 2) {
				uint4 hi, lo;
				const float h0 = (float)(__bf16)a.x, h1 = (float)(__bf16)a.y, h2 = (float)(__bf16)a.z,
					    h3 = (float)(__bf16)a.w, h4 = (float)(__bf16)c.x, h5 = (float)(__bf16)c.y,
					    h6 = (float)(__bf16)c.z, h7 = (float)(__bf16)c.w;
				hi = make_uint4(pack_bf16(h0, h1), pack_bf16(h2, h3), pack_bf16(h4, h5), pack_bf16(h6, h7));
				lo = make_uint4(pack_bf16(a.x - h0, a.y - h1), pack_bf16(a.z - h2, a.w - h3),
						pack_bf16(c.x - h4, c.y - h5), pack_bf16(c.z - h6, c.w - h7));
				reinterpret_cast<uint4 *>(r.xa + (size_t)t * r.d)[q / 2] = hi;
				reinterpret_cast<uint4 *>(r.xlo + (size_t)t * r.d)[q / 2] = lo;
			} else {
				reinterpret_cast<uint4 *>(r.xa + (size_t)t * r.d)[q / 2] =
					make_uint4(pack_bf16(a.x, a.y), pack_bf16(a.z, a.w), pack_bf16(c.x, c.y), pack_bf16(c.z, c.w));
			}
		}
	}
	if constexpr (MODE == 1) {
		bad = __any(bad);
		if (lane == 0) {
			r.flag[t] = bad;
			if (bad)
				r.list[atomicAdd(r.count, 1)] = t;
		}
	}
}

// Q4_K gate/up in 32-row tiles with the minimum term from the sub-block sums
// (exactly when the kernel instantiation's QF is on: it reads Workspace::xsum)
static bool mfma_gu_qfold(const Layer &L, int npairs)
{
	return Cfg<TIE_GGML_Q4_K, false, MFMA_MT_TINY>::UH && TIE_MFMA_QFOLD && L.gate.type == TIE_GGML_Q4_K &&
	       mfma_gu_rows(L, npairs) == MFMA_MT_TINY;
}

hipError_t launch_route_bucket(const Layer &L, const float *x, int T, int k, Workspace &ws, hipStream_t s,
			       bool converted)
{
	BucketArgs r;
	r.logits = ws.logits;
	r.T = T;
	r.ts = T4(T);
	r.E = L.E;
	r.k = k;
	r.d = L.d;
	r.routing = L.routing;
	r.pbias = L.pbias;
	r.topk_idx = ws.topk_idx;
	r.topk_w = ws.topk_w;
	r.sel = ws.sel;
	const bool append = route_appends(T);
	r.cnt = append ? ws.bucket_cnt : nullptr;
	r.bucket = append ? ws.bucket : nullptr;
	r.x = x;
	r.xa = ws.xb;
	r.xlo = ws.xlo;
	r.flag = ws.tok_flag;
	r.list = ws.fix_list;
	r.count = ws.fix_count;
	r.converted = converted && L.gate.type != TIE_GGML_BF16 && TIE_MFMA_F16;
	r.xsum = mfma_gu_qfold(L, T * k) ? ws.xsum : nullptr;
	const dim3 grid((T + RB_THREADS / 64 - 1) / (RB_THREADS / 64));
	if (L.gate.type == TIE_GGML_BF16)
		tie_launch(route_bucket_kernel<2>, grid, dim3(RB_THREADS), 0, s, r);
	else if (TIE_MFMA_F16)
		tie_launch(route_bucket_kernel<1>, grid, dim3(RB_THREADS), 0, s, r);
	else
		tie_launch(route_bucket_kernel<0>, grid, dim3(RB_THREADS), 0, s, r);
	return hipGetLastError();
}

hipError_t launch_bucket_plan(const Layer &L, int T, int k, Workspace &ws, hipStream_t s);

// Per-expert pair lists from the selection bytes, one workgroup per expert
// e: the tokens t with sel[e][t] = j + 1 != 0 in token order (ranks by an
// exclusive scan of each thread's count over 4 tokens per word): bucket[e]
// [rank] = t k + j, cnt[e] = their number.  No atomics: the expert kernels
// read the counts and their tiles' rows from here.
constexpr int BP_THREADS = 256;
__global__ __launch_bounds__(BP_THREADS) void bucket_plan_kernel(const uint8_t *__restrict__ sel, int k, int T,
								  int32_t *__restrict__ cnt, int32_t *__restrict__ bucket)
{
	__shared__ int wsum[BP_THREADS / 64];
	const int e = blockIdx.x, t = threadIdx.x;
	const uint32_t *row = reinterpret_cast<const uint32_t *>(sel + (size_t)e * T); // T % 4 == 0
	int32_t *bk = bucket + (size_t)e * T;
	const int nw = T / 4;
	int carry = 0;
	for (int w0 = 0; w0 < nw; w0 += 4 * BP_THREADS) {
		// 4 words (16 tokens) per thread
		uint32_t wd[4];
		int n = 0;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const int wi = w0 + 4 * t + i;
			wd[i] = wi < nw ? row[wi] : 0u;
#pragma unroll
			for (int b = 0; b < 4; b++)
				n += ((wd[i] >> (8 * b)) & 0xffu) ? 1 : 0;
		}
		int tot;
		int rk = carry + block_exclusive_scan<BP_THREADS>(n, wsum, tot);
#pragma unroll
		for (int i = 0; i < 4; i++)
#pragma unroll
			for (int b = 0; b < 4; b++) {
				const uint32_t v = (wd[i] >> (8 * b)) & 0xffu;
				if (v) {
					const int tok = 4 * (w0 + 4 * t + i) + b;
					bk[rk++] = tok * k + (int)v - 1;
				}
			}
		carry += tot;
	}
	if (t == 0)
		cnt[e] = carry;
}

hipError_t launch_bucket_plan(const Layer &L, int T, int k, Workspace &ws, hipStream_t s)
{
	tie_launch(bucket_plan_kernel, dim3(L.E), dim3(BP_THREADS), 0, s, ws.sel, k, T4(T), ws.bucket_cnt,
			   ws.bucket);
	return hipGetLastError();
}

template <int TYPE, bool DOWN, int MTR = 0>
static hipError_t launch_type(const MfmaArgs &a, dim3 grid, hipStream_t s)
{
	// the double-buffered A tile exceeds the default 64 KiB of dynamic LDS
	using C = Cfg<TYPE, DOWN, MTR>;
	constexpr size_t lds = (size_t)C::STAGE_BYTES + 4 * (size_t)(C::RPI * NWAVES * ROFF_STRIDE) + 4 * C::MT;
	static_assert(lds <= 160 * 1024, "LDS budget");
	static bool attr = false;
	if (!attr) {
		const hipError_t err = hipFuncSetAttribute((const void *)mfma_experts_kernel<TYPE, DOWN, MTR>,
							   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
		if (err != hipSuccess)
			return err;
		attr = true;
	}
	tie_launch((mfma_experts_kernel<TYPE, DOWN, MTR>), grid, dim3(MF_THREADS), lds, s, a);
	return hipGetLastError();
}

template <bool DOWN>
static hipError_t launch_one(const MfmaArgs &a, int type, dim3 grid, hipStream_t s, int mt = 0)
{
	if constexpr (!DOWN) {
		if (mt == MFMA_MT_TINY && type == TIE_GGML_Q4_K)
			return launch_type<TIE_GGML_Q4_K, false, MFMA_MT_TINY>(a, grid, s);
		if (mt == MFMA_MT_TINY && type == TIE_GGML_Q6_K)
			return launch_type<TIE_GGML_Q6_K, false, MFMA_MT_TINY>(a, grid, s);
		if (mt == MFMA_MT_GU_SMALL && type == TIE_GGML_Q4_K)
			return launch_type<TIE_GGML_Q4_K, false, MFMA_MT_GU_SMALL>(a, grid, s);
		if (mt == MFMA_MT_GU_SMALL && type == TIE_GGML_Q6_K)
			return launch_type<TIE_GGML_Q6_K, false, MFMA_MT_GU_SMALL>(a, grid, s);
	} else {
		if (mt == MFMA_MT_TINY && type == TIE_GGML_Q4_K)
			return launch_type<TIE_GGML_Q4_K, true, MFMA_MT_TINY>(a, grid, s);
		if (mt == MFMA_MT_TINY && type == TIE_GGML_Q6_K)
			return launch_type<TIE_GGML_Q6_K, true, MFMA_MT_TINY>(a, grid, s);
	}
	if (type == TIE_GGML_Q4_K)
		return launch_type<TIE_GGML_Q4_K, DOWN>(a, grid, s);
	if (type == TIE_GGML_Q6_K)
		return launch_type<TIE_GGML_Q6_K, DOWN>(a, grid, s);
	return launch_type<TIE_GGML_BF16, DOWN>(a, grid, s);
}

bool mfma_f16_operands(const Layer &L)
{
	const bool q = L.gate.type == TIE_GGML_Q4_K || L.gate.type == TIE_GGML_Q6_K;
	const bool qd = L.down.type == TIE_GGML_Q4_K || L.down.type == TIE_GGML_Q6_K;
	return TIE_MFMA_F16 && (q || qd);
}

// Quantised gate/up with at most TIE_MFMA_SMALL_AVG pairs per expert on
// average: 64-row tiles, three waves per SIMD (smaller accumulator and LDS
// footprint); measured faster there, slower for large expert counts.
int mfma_gu_rows(const Layer &L, int npairs)
{
	const bool quant = L.gate.type == TIE_GGML_Q4_K || L.gate.type == TIE_GGML_Q6_K;
	if (quant && npairs <= TIE_MFMA_TINY_AVG * L.E)
		return MFMA_MT_TINY;
	if (!quant)
		return MFMA_MT_GU_BF16;
	return npairs <= TIE_MFMA_SMALL_AVG * L.E ? MFMA_MT_GU_SMALL : MFMA_MT_GU;
}

// Quantised down with at most TIE_MFMA_TINY_AVG pairs per expert on average:
// 32-row tiles, whose small activation buffers leave the LDS for more
// weight stages in flight (decode-sized batches stream the weights).
int mfma_dn_rows(const Layer &L, int npairs)
{
	const bool quant = L.down.type == TIE_GGML_Q4_K || L.down.type == TIE_GGML_Q6_K;
	if (!quant)
		return MFMA_MT_DN_BF16;
	return npairs <= TIE_MFMA_TINY_AVG * L.E ? MFMA_MT_TINY : MFMA_MT_DN;
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
	(void)x;
	// the kernels address activation rows with 32-bit byte offsets; tiles
	// are GU_COLS gate/up and DN_COLS down columns wide
	if ((size_t)T * L.d * 4 > 0xfffffffeu || (size_t)npairs * L.F * 4 > 0xfffffffeu || L.F % GU_COLS ||
	    L.d % DN_COLS)
		return hipErrorInvalidValue;
	MfmaArgs a;
	memset(&a, 0, sizeof a);
	a.k = k;
	a.E = L.E;
	a.cnt = ws.bucket_cnt;
	a.bucket = ws.bucket;
	a.bstride = T4(T);
	a.silu = silu;
	a.y = ws.y;
	a.h_f16 = TIE_MFMA_F16 && (L.down.type == TIE_GGML_Q4_K || L.down.type == TIE_GGML_Q6_K);
	a.y16 = TIE_MFMA_Y16 && a.h_f16 ? reinterpret_cast<uint16_t *>(ws.y) : nullptr;
	a.h_scale = ldexpf(1.0f, -L.h_shift);
	a.y_scale = ldexpf(1.0f, L.h_shift - F16_SHIFT - (a.y16 ? L.y_shift : 0));
	a.tok_flag = ws.tok_flag;
	a.fix_list = ws.fix_list;
	a.fix_count = ws.fix_count;
	// grid rows: a bound on each kernel's tiles (its own tile rows) plus 8
	// rows: the XCD remap in the kernel reaches every live item only with
	// at least 8 * ceil(live / 8) workgroups (rows past the tiles exit at
	// once)
	const int mt_gu = mfma_gu_rows(L, npairs), mt_dn = mfma_dn_rows(L, npairs);
	// decode-sized batches: one item per (expert, slab) and h by expert
	// (both kernels of 32-row tiles, f16 h, the workspace's expert-major h)
	a.direct = TIE_MFMA_DIRECT && mt_gu == MFMA_MT_TINY && mt_dn == MFMA_MT_TINY && T <= MFMA_DIRECT_T &&
		   a.h_f16 && ws.hd != nullptr;
	const int gu_tiles = a.direct ? L.E + 8 : (npairs + mt_gu - 1) / mt_gu + L.E + 8;
	const int dn_tiles = a.direct ? L.E + 8 : (npairs + mt_dn - 1) / mt_dn + L.E + 8;
	uint16_t *hrows = a.direct ? ws.hd : ws.hb;

	prof_begin("mfma_gate_up", s);
	a.w[0] = L.gate.data;
	a.w[1] = L.up.data;
	a.expert_bytes[0] = L.gate.expert_bytes;
	a.expert_bytes[1] = L.up.expert_bytes;
	a.rows = L.F;
	a.in = L.d;
	a.a16 = ws.xb;
	a.a16lo = ws.xlo;
	a.xsum = mfma_gu_qfold(L, npairs) ? ws.xsum : nullptr;
	a.h16 = hrows;
	a.h16lo = ws.hlo;
	hipError_t err = launch_one<false>(a, L.gate.type, dim3(L.F / GU_COLS, gu_tiles), s, mt_gu);
	prof_end(s);
	if (err != hipSuccess)
		return err;

	prof_begin("mfma_down", s);
	a.w[0] = a.w[1] = L.down.data;
	a.expert_bytes[0] = a.expert_bytes[1] = L.down.expert_bytes;
	a.rows = L.d;
	a.in = L.F;
	a.a16 = hrows;
	a.a16lo = ws.hlo;
	if (split_down && !split) {
		prof_end(s);
		return hipErrorInvalidValue; // h has no remainder plane for the split down path
	}
	err = launch_one<true>(a, L.down.type, dim3(L.d / DN_COLS, dn_tiles), s, mt_dn);
	prof_end(s);
	return err;
}

// ------------------------------------------------------------ dense matrices
// dispatch_mat_mat (math_dispatch.c:304-359) on the f16 matrix cores: the
// matrix is one "expert" whose pairs are the T tokens in order (k = 1), run
// by the down kernel (A = x as f16 in the pair-permuted K order, unscaled;
// fp32 output rows).  dense_prep_kernel converts x (one wave per token),
// flags tokens whose x leaves the f16 range (their rows are recomputed in
// TIE's exact arithmetic afterwards, launch_dense_fix), and writes the
// one-expert pair list (cnt[0] = T, bucket[t] = t).
__global__ __launch_bounds__(RB_THREADS) void dense_prep_kernel(const float *__restrict__ x, int T, int in,
								 uint16_t *__restrict__ xa, int32_t *__restrict__ cnt,
								 int32_t *__restrict__ bucket, int32_t *__restrict__ flag)
{
	const int lane = threadIdx.x & 63;
	const int t = blockIdx.x * (RB_THREADS / 64) + (threadIdx.x >> 6);
	if (t >= T)
		return;
	if (t == 0 && lane == 0)
		cnt[0] = T;
	if (lane == 0)
		bucket[t] = t;
	const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)t * in);
	f16x8 *yr = reinterpret_cast<f16x8 *>(xa + (size_t)t * in);
	int bad = 0;
	for (int i = lane; i < in / 8; i += 64) {
		const float4 a = xr[2 * i], c = xr[2 * i + 1];
		const float m = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(a.x), __builtin_fabsf(a.y)),
								__builtin_fmaxf(__builtin_fabsf(a.z), __builtin_fabsf(a.w))),
						__builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(c.x), __builtin_fabsf(c.y)),
								__builtin_fmaxf(__builtin_fabsf(c.z), __builtin_fabsf(c.w))));
		// fmax drops NaN: test the values themselves for NaN
		const bool nan = a.x != a.x || a.y != a.y || a.z != a.z || a.w != a.w || c.x != c.x || c.y != c.y ||
				 c.z != c.z || c.w != c.w;
		bad |= (nan || !(m < 65504.0f)) ? 1 : 0;
		yr[i] = f16x8{(_Float16)a.x, (_Float16)a.z, (_Float16)a.y, (_Float16)a.w,
			      (_Float16)c.x, (_Float16)c.z, (_Float16)c.y, (_Float16)c.w};
	}
	bad = __any(bad);
	if (lane == 0)
		flag[t] = bad;
}

bool mfma_dense_supported(const ExpertTensor &W, int T)
{
	return TIE_MFMA_F16 && (W.type == TIE_GGML_Q4_K || W.type == TIE_GGML_Q6_K) && W.rows % DN_COLS == 0 &&
	       (size_t)T * W.in * 2 <= 0xfffffffeu && (size_t)T * W.rows * 4 <= 0xfffffffeu;
}

hipError_t launch_mfma_dense(const ExpertTensor &W, const float *x, int T, float *out, Workspace &ws, hipStream_t s)
{
	if (T == 0)
		return hipSuccess;
	if (!mfma_dense_supported(W, T))
		return hipErrorInvalidValue;
	tie_launch(dense_prep_kernel, dim3((T + RB_THREADS / 64 - 1) / (RB_THREADS / 64)), dim3(RB_THREADS), 0, s, x,
			   T, W.in, ws.xb, ws.bucket_cnt, ws.bucket, ws.tok_flag);
	hipError_t err = hipGetLastError();
	if (err != hipSuccess)
		return err;
	MfmaArgs a;
	memset(&a, 0, sizeof a);
	a.k = 1;
	a.E = 1;
	a.cnt = ws.bucket_cnt;
	a.bucket = ws.bucket;
	a.bstride = T4(T);
	a.y_scale = ldexpf(1.0f, -F16_SHIFT); // x unscaled; the weights' factor 2^F16_SHIFT out
	a.y = out;
	a.w[0] = a.w[1] = W.data;
	a.expert_bytes[0] = a.expert_bytes[1] = W.expert_bytes;
	a.rows = W.rows;
	a.in = W.in;
	a.a16 = ws.xb;
	// tiles of fewer rows while the matrix's column slabs alone leave CUs
	// idle (each tile then dequantises its slab again, from the cache)
	const int slabs = W.rows / DN_COLS;
	int mt = MFMA_MT_DN;
	while (mt > 32 && slabs * ((T + mt - 1) / mt) < 256)
		mt >>= 1;
	a.mt_cap = mt;
	const int tiles = (T + mt - 1) / mt + 1 + 8;
	err = launch_one<true>(a, W.type, dim3(W.rows / DN_COLS, tiles), s);
	if (err != hipSuccess)
		return err;
	return launch_dense_fix(W, x, T, out, ws.tok_flag, s);
}

} // namespace tie

#ifdef TIE_MFMA_TIMELINE
extern "C" int tie_hip_debug_mfma_timeline(unsigned long long *host, int reset)
{
	const size_t n = sizeof(unsigned long long) * 2 * tie::MFMA_TL_WG * 2;
	if (hipMemcpyFromSymbol(host, HIP_SYMBOL(tie::g_mfma_tl), n) != hipSuccess)
		return -1;
	if (reset) {
		static unsigned long long z[2 * tie::MFMA_TL_WG * 2];
		if (hipMemcpyToSymbol(HIP_SYMBOL(tie::g_mfma_tl), z, n) != hipSuccess)
			return -1;
	}
	return 0;
}
#endif

#ifdef TIE_MFMA_TRACE
extern "C" int tie_hip_debug_mfma_trace(unsigned long long *host, int reset)
{
	if (hipMemcpyFromSymbol(host, HIP_SYMBOL(tie::g_mfma_trace), sizeof(unsigned long long) * 16) != hipSuccess)
		return -1;
	if (reset) {
		static const unsigned long long z[16] = {0};
		if (hipMemcpyToSymbol(HIP_SYMBOL(tie::g_mfma_trace), z, sizeof z) != hipSuccess)
			return -1;
	}
	return 0;
}
#endif

