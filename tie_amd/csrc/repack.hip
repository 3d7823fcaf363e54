// repack.hip -- one-time conversion of GGUF expert tensors to the device
// panel layout (see ExpertTensor in common.h).
//
// Source layout (gguf.h:100-113, process_expert_task's offsets at
// engine.c:929-950): stacked [E][rows][in]; a quantised row is in/256
// consecutive super-blocks; BF16 rows are in consecutive bf16.
#include "common.h"

namespace tie {

// Q4_K: one thread per (block, 16-byte chunk).  Blocks are 144 bytes, so a
// 16-byte aligned source keeps every chunk aligned.
__global__ void repack_q4k_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int E, int rows,
				  int nb, size_t expert_bytes, int aligned)
{
	const size_t total = (size_t)E * rows * nb * Q4K_CHUNKS;
	for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
		const size_t blk = g / Q4K_CHUNKS;
		const int c = (int)(g % Q4K_CHUNKS);
		const int b = (int)(blk % nb);
		const size_t er = blk / nb; // e * rows + r
		const int r = (int)(er % rows);
		const int e = (int)(er / rows);
		const int rt = r / PANEL_ROWS, i = r % PANEL_ROWS;
		uint8_t *d = dst + (size_t)e * expert_bytes + (((size_t)rt * nb + b) * Q4K_CHUNKS + c) * 1024 + i * 16;
		const uint8_t *s = src + blk * Q4K_BYTES + c * 16;
		if (aligned) {
			*reinterpret_cast<uint4 *>(d) = *reinterpret_cast<const uint4 *>(s);
		} else {
			for (int q = 0; q < 16; q++)
				d[q] = s[q];
		}
	}
}

// Q6_K: one thread per block; ql -> chunks 0-7, qh -> 8-11, scales -> 12,
// d -> the fp16 plane after the 13 chunks.
__global__ void repack_q6k_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int E, int rows,
				  int nb, size_t expert_bytes)
{
	const size_t total = (size_t)E * rows * nb;
	for (size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x; blk < total;
	     blk += (size_t)gridDim.x * blockDim.x) {
		const int b = (int)(blk % nb);
		const size_t er = blk / nb;
		const int r = (int)(er % rows);
		const int e = (int)(er / rows);
		const int rt = r / PANEL_ROWS, i = r % PANEL_ROWS;
		uint8_t *panel = dst + (size_t)e * expert_bytes + ((size_t)rt * nb + b) * Q6K_PANEL;
		const uint8_t *s = src + blk * Q6K_BYTES;
		for (int c = 0; c < Q6K_CHUNKS; c++) {
			uint8_t *d = panel + c * 1024 + i * 16;
			for (int q = 0; q < 16; q++)
				d[q] = s[16 * c + q]; // ql[0..127] | qh[0..63] | scales[16] are contiguous in the block
		}
		panel[Q6K_CHUNKS * 1024 + 2 * i] = s[208];
		panel[Q6K_CHUNKS * 1024 + 2 * i + 1] = s[209];
	}
}

// BF16: copy expert e from its source offset into a contiguous [rows][in]
// slot.  literal != 0 takes expert e at e*rows*(in/256)*2 bytes, the offset
// process_expert_task computes with ggml_block_size(BF16) = 2
// (engine.c:929-942, gguf.c:28-29).
__global__ void repack_bf16_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int E, int rows,
				   int in, int literal)
{
	const size_t per = (size_t)rows * in * 2; // bytes per expert
	const size_t total = (size_t)E * per / 2; // 16-bit elements
	for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (size_t)gridDim.x * blockDim.x) {
		const size_t e = g / (per / 2);
		const size_t o = g % (per / 2);
		const size_t src_off = literal ? e * (size_t)rows * (in / 256) * 2 : e * per;
		const uint8_t *s = src + src_off + 2 * o;
		uint8_t *d = dst + e * per + 2 * o;
		d[0] = s[0];
		d[1] = s[1];
	}
}

hipError_t launch_repack(const ExpertTensor &t, const uint8_t *src, int E, int literal_bf16_stride, hipStream_t s)
{
	uint8_t *dst = const_cast<uint8_t *>(t.data);
	const int threads = 256, blocks = 4096;
	if (t.type == TIE_GGML_Q4_K) {
		const int aligned = ((uintptr_t)src % 16) == 0;
		tie_launch(repack_q4k_kernel, dim3(blocks), dim3(threads), 0, s, src, dst, E, t.rows, t.nb,
				   t.expert_bytes, aligned);
	} else if (t.type == TIE_GGML_Q6_K) {
		tie_launch(repack_q6k_kernel, dim3(blocks), dim3(threads), 0, s, src, dst, E, t.rows, t.nb,
				   t.expert_bytes);
	} else if (t.type == TIE_GGML_BF16) {
		tie_launch(repack_bf16_kernel, dim3(blocks), dim3(threads), 0, s, src, dst, E, t.rows, t.in,
				   literal_bf16_stride);
	} else {
		return hipErrorInvalidValue;
	}
	return hipGetLastError();
}

} // namespace tie
