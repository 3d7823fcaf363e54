/*
 * tie_hip.h -- C ABI of the MI355X (gfx950) Qwen3-MoE FFN block for TIE.
 *
 * The reference (szemzoa/tie) runs the MoE FFN inline in
 * transformer_layer_qwen3 (model_qwen3.c:404-471): per token a router GEMV
 * (dispatch_mat_vec, model_qwen3.c:431-432), find_top_k (engine.c:891),
 * softmax over the k selected logits (engine.c:864), k process_expert_task
 * jobs on the thread pool (engine.c:916-964) and an fp32 weighted combine
 * (model_qwen3.c:459-470).  This library replaces that whole branch with
 * HIP kernels.  Every entry point is plain C: pointers, sizes and GGML type
 * ids (gguf.h:8-36), no HIP or torch types.
 *
 * Return codes: 0 on success, a negative TIE_HIP_E* code otherwise; the
 * library never exits the process.  tie_hip_last_error() describes the
 * last failure of the calling thread.
 */
#ifndef TIE_HIP_H
#define TIE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TIE_HIP_ABI_VERSION 2

/* GGML type ids as in gguf.h:8-36 */
#define TIE_GGML_F32 0
#define TIE_GGML_Q4_K 12
#define TIE_GGML_Q6_K 14
#define TIE_GGML_BF16 30

#define TIE_HIP_OK 0
#define TIE_HIP_EINVAL (-1)  /* bad argument, shape or type (TIE: return -1, model_qwen3.c:407-410) */
#define TIE_HIP_EHIP (-2)    /* a HIP runtime error */
#define TIE_HIP_ENOMEM (-3)  /* device allocation failed */
#define TIE_HIP_ENOINIT (-4) /* tie_hip_init() not called */

#define TIE_SILU_TABLE_SIZE 8192 /* SILU_TABLE_SIZE, engine.h:10 */

/* Forward flags */
#define TIE_HIP_PATH_AUTO 0x0  /* exact fp32 GEMV path up to tie_hip_exact_max_tokens() (21), 16-bit MFMA grouped GEMM above */
#define TIE_HIP_PATH_EXACT 0x1 /* always the fp32 path that reproduces TIE's arithmetic bit for bit */
#define TIE_HIP_PATH_MFMA 0x2  /* always the grouped-GEMM path */

/* Routing modes (tie_hip_layer_desc.routing) */
#define TIE_HIP_ROUTE_SOFTMAX 0 /* Qwen3: top-k of the logits, softmax over the k (model_qwen3.c:431-443) */
#define TIE_HIP_ROUTE_SIGMOID 1 /* LFM2: sigmoid, top-k of sigmoid + bias, L1-normalised sigmoid of the k
				   (model_lfm2.c:437-467) */

typedef struct tie_hip_layer tie_hip_layer;

/* Library set-up on one HIP device; replaces the MoE-relevant part of
 * engine_alloc (engine.c:14-40: thread pool, silu_table_init,
 * math_dispatch_init).  Builds the SiLU table on the host CPU the way TIE
 * does and uploads it. */
int tie_hip_init(int device);

/* Frees every device resource, including the weight cache. */
void tie_hip_shutdown(void);

/* Text of the last error on the calling thread ("" when none). */
const char *tie_hip_last_error(void);

/* Drop-in for the MoE branch of transformer_layer_qwen3
 * (model_qwen3.c:404-471).  Host pointers, as TIE holds them:
 *   x          ctx->mem.normed_ffn_input, [T][d] F32
 *   router_w   ffn_gate_inp, F32 [E][d] (router_type must be TIE_GGML_F32)
 *   gate/up    ffn_{gate,up}_exps, [E][F][d] in GGUF block layout
 *   down       ffn_down_exps, [E][d][F] in GGUF block layout
 *   out        ctx->mem.ffn_down_output, [T][d] F32
 *   topk_idx_opt / topk_w_opt  optional [T][k] selected experts / weights
 * Expert types: TIE_GGML_Q4_K, TIE_GGML_Q6_K or TIE_GGML_BF16.  d and F must
 * be multiples of 256, k <= E <= 1024, k <= 32.  Weight tensors are uploaded
 * once and cached, keyed by host pointer, type and size (they must stay
 * valid and unchanged while cached, as TIE's mmap'd weights are).  Runs on
 * the library's stream and returns after out is written. */
int tie_hip_moe_ffn(const float *x, int T, int d, int F, int E, int k, const void *router_w, int router_type,
		    const void *gate_exps, int gate_type, const void *up_exps, int up_type, const void *down_exps,
		    int down_type, float *out, int32_t *topk_idx_opt, float *topk_w_opt);

/* Drop-in for the MoE branch of transformer_layer_lfm2
 * (model_lfm2.c:414-497).  Same arguments as tie_hip_moe_ffn plus
 *   probs_bias_opt  exp_probs_b_bias, F32 [E] host array, or NULL (the
 *                   branch at model_lfm2.c:446-454)
 * Routing is TIE_HIP_ROUTE_SIGMOID: p_e = 1/(1+expf(-logit_e)), top-k of
 * p_e + bias_e, weights p_j / (sum_j p_j + 1e-6); the experts and the
 * combine are those of tie_hip_moe_ffn. */
int tie_hip_moe_ffn_lfm2(const float *x, int T, int d, int F, int E, int k, const void *router_w, int router_type,
			 const float *probs_bias_opt, const void *gate_exps, int gate_type, const void *up_exps,
			 int up_type, const void *down_exps, int down_type, float *out, int32_t *topk_idx_opt,
			 float *topk_w_opt);

/* Drop-in for the whole FFN half of transformer_layer_qwen3 (the RMSNorm at
 * model_qwen3.c:392-401, the MoE branch at :404-471 and the residual add at
 * :491): hidden += MoE(rms_norm(hidden, ffn_norm, eps)).
 *   hidden    ctx->mem.hidden_state, [T][d] F32, read and updated in place
 *   ffn_norm  LayerWeights.ffn_norm (engine.h:72), F32 [d]
 *   eps       ctx->model->norm_eps
 * The RMSNorm reproduces rms_norm_f32_f32_f32_avx2 (math_avx2.c:56-96) as
 * TIE's build computes it, including the host CPU's RSQRTSS approximation
 * (tabulated on this host at the first call).  Other arguments as
 * tie_hip_moe_ffn. */
int tie_hip_qwen3_ffn(float *hidden, int T, int d, int F, int E, int k, const float *ffn_norm, float eps,
		      const void *router_w, int router_type, const void *gate_exps, int gate_type, const void *up_exps,
		      int up_type, const void *down_exps, int down_type, int32_t *topk_idx_opt, float *topk_w_opt);

/* Replace the SiLU lookup table with the caller's (TIE's own silu_table,
 * engine.c:12, as filled by silu_table_init, engine.c:297-303). */
int tie_hip_set_silu_table(const float *table, int n);

/* Build the SiLU table on the host CPU exactly as TIE's compiled
 * silu_table_init does on this host (no GPU needed). */
int tie_hip_silu_table_host(float *table, int n);

/* ------------------------------------------------------------------ */
/* Device-resident layers (inputs already in HBM)                       */
/* ------------------------------------------------------------------ */

typedef struct tie_hip_layer_desc {
	int d, F, E;
	const void *router_w; /* F32 [E][d] */
	int router_type;      /* TIE_GGML_F32 */
	const void *gate_exps;
	int gate_type;
	const void *up_exps;
	int up_type;
	const void *down_exps;
	int down_type;
	const float *router_bias; /* optional [E], added to the logits before top-k; NULL in TIE */
	int src_on_device;        /* 1: the pointers above are device memory (GGUF layout); the
				     library drains the device before reading them, so work on any
				     stream that writes them has finished */
	int literal_bf16_stride;  /* 1: BF16 experts start at e*rows*(in/256)*2 bytes, as
				     process_expert_task computes it (engine.c:929-942) */
	int routing;              /* TIE_HIP_ROUTE_SOFTMAX (0, Qwen3) or TIE_HIP_ROUTE_SIGMOID (LFM2) */
	const float *probs_bias;  /* optional [E]: LFM2's exp_probs_b_bias, added to the sigmoid
				     scores for the selection only (ROUTE_SIGMOID) */
} tie_hip_layer_desc;

/* Upload (or copy on device) and repack one layer's weights into the
 * device layout.  The source buffers may be freed afterwards.  With
 * src_on_device (and for tie_hip_matrix_create likewise) the library drains
 * the device (hipDeviceSynchronize): no thread may be capturing a HIP graph
 * meanwhile, as a device synchronisation fails or invalidates a capture in
 * global or relaxed mode. */
int tie_hip_layer_create(const tie_hip_layer_desc *desc, tie_hip_layer **out);
void tie_hip_layer_destroy(tie_hip_layer *layer);

/* Device bytes held by a layer. */
size_t tie_hip_layer_bytes(const tie_hip_layer *layer);

/* MoE block on device pointers, enqueued on `stream` (a hipStream_t; NULL =
 * the library stream).  x_dev/out_dev are [T][d] F32; topk outputs are
 * optional [T][k].  Returns once enqueued; the caller synchronises.
 *
 * Streams: the library keeps one scratch workspace per stream, so forwards
 * enqueued on different streams never share scratch memory and may run
 * concurrently (on distinct out buffers).  Forwards on one stream are
 * ordered by that stream.  When a call needs a larger workspace than its
 * stream holds, the library drains the whole device (hipDeviceSynchronize)
 * before freeing the old one; a call made during HIP graph capture must
 * therefore not grow it (warm the stream up with the largest T first).
 *
 * One token (T = 1, eager) runs as one launch whose workgroups hand values
 * to each other; their waits are bounded.  Should a wait give up (the GPU
 * did not run the workgroups together, e.g. under heavy sharing), that
 * call's outputs are NaN and the stream's status word is set: the
 * synchronous entry points (tie_hip_moe_ffn, _lfm2, tie_hip_qwen3_ffn)
 * then return TIE_HIP_EHIP, and device-API callers read it with
 * tie_hip_stream_status. */
/* Frees the scratch workspace the library keeps for `stream` (grown by the
 * forwards enqueued on it; at the 235B shape and large T, hundreds of MiB).
 * Call it before destroying a stream that forwards ran on; otherwise the
 * workspace lives until tie_hip_shutdown.  Drains the device first. */
int tie_hip_stream_release(void *stream);

int tie_hip_moe_forward(tie_hip_layer *layer, const float *x_dev, int T, int k, float *out_dev,
			int32_t *topk_idx_dev, float *topk_w_dev, int flags, void *stream);

/* tie_hip_moe_forward that allocates nothing: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  Its
 * scratch is one static 24 MiB device array per GPU (held until the process
 * ends) instead of the per-stream workspace: calls whose scratch would not
 * fit (T * k pairs with this layer's shape: T <= 89 at d = 2048, F = 768,
 * k = 8; T <= 44 at d = 4096, F = 1536, k = 8) return TIE_HIP_EINVAL.  All calls on a GPU share the array,
 * so calls that overlap in time on one GPU (other streams, other threads)
 * race: serialise them.  Same arguments, results and stream rules as
 * tie_hip_moe_forward otherwise. */
int tie_hip_moe_forward_noalloc(tie_hip_layer *layer, const float *x_dev, int T, int k, float *out_dev,
				int32_t *topk_idx_dev, float *topk_w_dev, int flags, void *stream);

/* The same FFN half on device pointers: out_dev = hidden_dev +
 * block(rms_norm(hidden_dev)), both [T][d] F32; out_dev may be hidden_dev
 * (TIE's in-place update).  ffn_norm_dev [d] F32.  Enqueued on `stream` like
 * tie_hip_moe_forward. */
int tie_hip_moe_forward_residual(tie_hip_layer *layer, const float *hidden_dev, const float *ffn_norm_dev, float eps,
				 int T, int k, float *out_dev, int32_t *topk_idx_dev, float *topk_w_dev, int flags,
				 void *stream);

/* ------------------------------------------------------------------ */
/* Dense matrices (dispatch_mat_mat with F32 input)                     */
/* ------------------------------------------------------------------ */

typedef struct tie_hip_matrix tie_hip_matrix;

/* Upload one GGUF weight matrix [rows][in_dim] (ne = [in_dim, rows]) of type
 * TIE_GGML_F32, Q4_K, Q6_K or BF16 (repacked into the panel layout); rows a
 * multiple of 64, in_dim a multiple of 256 up to 16384.  The source may be
 * freed afterwards. */
int tie_hip_matrix_create(const void *w, int type, int rows, int in_dim, int src_on_device, tie_hip_matrix **out);
void tie_hip_matrix_destroy(tie_hip_matrix *m);

/* dispatch_mat_mat (math_dispatch.c:304-359) on device pointers:
 * out_dev[t][r] = W[r] . x_dev[t] for t < T, x [T][in_dim] F32, out
 * [T][rows] F32.  TIE_HIP_PATH_EXACT and TIE_HIP_PATH_AUTO (the default, at
 * every T) use TIE's row kernels (mat_vec_row_f32_{f32,q4k,q6k,
 * bf16}_f32_avx2) bit for bit.  TIE_HIP_PATH_MFMA (opt-in; Q4_K or Q6_K,
 * rows a multiple of 256) runs the f16 matrix cores with fp32 accumulation
 * (relative L2 error about 3e-4 of TIE's result); rows whose input does not
 * fit the f16 range are recomputed with the exact kernel.
 * TIE_HIP_PATH_MFMA on an unsupported matrix is an error.  Enqueued on `stream`.  The attention projections, the dense FFN and the LM
 * head of transformer_layer_qwen3 / main.c use it. */
int tie_hip_mat_mat(tie_hip_matrix *m, const float *x_dev, int T, float *out_dev, int flags, void *stream);

/* ------------------------------------------------------------------ */
/* GGUF models: every MoE layer uploaded once                           */
/* ------------------------------------------------------------------ */

typedef struct tie_hip_model_info {
	char architecture[32]; /* general.architecture */
	int d, F, E, k;        /* embedding_length, expert_feed_forward_length, expert_count, expert_used_count */
	int n_layers;          /* block_count */
	int first_moe_layer;   /* leading_dense_block_count (LFM2), else 0 */
	float norm_eps;        /* attention.layer_norm_rms_epsilon */
	int routing;           /* TIE_HIP_ROUTE_SIGMOID for LFM2, else TIE_HIP_ROUTE_SOFTMAX */
} tie_hip_model_info;

typedef struct tie_hip_model tie_hip_model;

/* Read the MoE shape of a GGUF file (host only, no GPU needed). */
int tie_hip_gguf_inspect(const char *path, tie_hip_model_info *info);

/* One tensor as the library's reader maps it (host only): its GGML type,
 * ne[0..3] (GGUF order, 1 past n_dims), the file offset of its data (the
 * data section starts at the first multiple of general.alignment, default
 * 32, after the tensor infos: gguf_model_map_weights, gguf.c:941-944) and
 * its size in bytes (0 for types the MoE path does not read).  name NULL:
 * only the count.  Returns the file's tensor count, or a negative code. */
int tie_hip_gguf_tensor_info(const char *path, const char *name, int *type, uint64_t ne[4], uint64_t *file_offset,
			     uint64_t *bytes);

/* Map a GGUF file and upload the MoE FFN of every layer from
 * first_moe_layer on: blk.N.ffn_gate_inp / ffn_gate_exps / ffn_up_exps /
 * ffn_down_exps (and exp_probs_b.bias for LFM2) into a tie_hip_layer, and
 * blk.N.ffn_norm.weight to the device, as TIE's model loading maps them
 * (gguf_model_map_weights, gguf.c:892-966; model_load_tensor, model.c:198-235).
 * The file is unmapped before returning. */
int tie_hip_gguf_load(const char *path, tie_hip_model **out);
void tie_hip_model_info_get(const tie_hip_model *m, tie_hip_model_info *info);
/* Layer n's block (NULL for a dense layer) and its device ffn_norm [d] (NULL
 * when the file has none). */
tie_hip_layer *tie_hip_model_layer(tie_hip_model *m, int n);
const float *tie_hip_model_ffn_norm(const tie_hip_model *m, int n);
void tie_hip_model_close(tie_hip_model *m);

/* The largest T that TIE_HIP_PATH_AUTO sends down the exact path (default
 * 14: from 15 tokens on the matrix-core path is the faster one at the 30B shape;
 * 64 or more keeps every decode-sized batch bit-exact). */
int tie_hip_exact_max_tokens(void);
void tie_hip_set_exact_max_tokens(int t);

/* Synchronises `stream` (NULL = the library stream) and reports whether a
 * one-token forward enqueued on it since the last check had a wait between
 * workgroups give up (its outputs NaN): TIE_HIP_EHIP with a message, and
 * the flag cleared; TIE_HIP_OK otherwise.  No counterpart in TIE (its CPU
 * path cannot fail this way). */
int tie_hip_stream_status(void *stream);

/* Debug hook: the next n one-launch one-token forwards wait for a stamp no
 * workgroup writes, with a 64-poll limit, so every wait gives up (and every
 * workgroup still exits): the error path of tie_hip_stream_status. */
void tie_hip_debug_decode_give_up(int n);

/* Debug: force the one-launch one-token kernel's form -- 0 a lane per
 * (row, block) dot, 1 two lanes per dot where the shape's block size and LDS
 * allow them; -1 chosen by the shape (two lanes when every workgroup fits
 * at once).  Both forms give the same bits. */
void tie_hip_debug_decode_form(int form);

/* Debug: the powers of two the layer's matrix-core path scales h and y by
 * (h stored as f16(h 2^-h_shift), y as f16(y 2^-y_shift)), chosen at
 * upload from samples of the gate and down weights. */
int tie_hip_debug_layer_shifts(const tie_hip_layer *layer, int *h_shift, int *y_shift);

/* Make the n-th next device allocation fail with TIE_HIP_ENOMEM (n >= 1;
 * 0 disarms).  Host-side fault injection for error-path tests. */
void tie_hip_debug_fail_alloc(int n);

/* Per-kernel timing: while enabled, every kernel of a named section (router,
 * dispatch, expert kernels, combine, ...) is launched with a start and stop
 * event bound to its own dispatch (hipExtLaunchKernel): a section's time is
 * the sum of its kernels' execution times.  Enabling (or disabling) clears
 * what was collected. */
int tie_hip_profile_enable(int on);

/* Sum of event-timed durations and section count per kernel name since the
 * last tie_hip_profile_enable(1); names come back comma-separated in
 * `names`.  Synchronises the device.  Returns the number of names. */
int tie_hip_profile_read(char *names, size_t names_cap, double *total_ms, int *launches, int max_kernels);

/* Host build of the device expf (tie_expf.h) over n inputs, for checking
 * it against the host libm (no GPU needed). */
void tie_hip_host_expf(const float *in, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
