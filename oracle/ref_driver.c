/*
 * ref_driver.c -- drives the compiled reference (szemzoa/tie) MoE path.
 *
 * TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together
 * with the reference's own sources, where they lie under /root/reference,
 * into oracle/_ref/libtie_ref.so.  It is used to pin the C restatement
 * (tie_oracle.c) with golden vectors and as the CPU baseline of bench.py.
 *
 * The reference has no standalone MoE function: the block is inline in
 * transformer_layer_qwen3 (model_qwen3.c:404-471).  ref_moe_block() sets up
 * the minimum of a TIEContext (Model with one LayerWeights, the MoE scratch
 * of model.c:416-433, the global thread pool of engine.c:23-24, the SiLU
 * table and the dispatch cache of engine.c:35-39) and then runs the same
 * per-token sequence as model_qwen3.c:415-471 by calling the reference's
 * own dispatch_mat_vec, find_top_k, softmax, process_expert_task and
 * dispatch_convert.
 *
 * routing == 1 runs the LFM2 selection of model_lfm2.c:437-467 instead
 * (sigmoid, optional exp_probs_b_bias for the selection, L1-normalised
 * weights), restated here over the reference's find_top_k, compiled with
 * the reference's flags so the sigmoid and sum loops vectorise as TIE's do.
 *
 * Two harness extensions, both off by default:
 *   router_bias  -- added to the router logits before top-k (the Zipf
 *                   routing config; TIE's Qwen3 path has no router bias);
 *   literal_bf16_stride == 0 with BF16 experts -- the expert task below
 *                   computes the expert byte offset as rows*in*2 instead of
 *                   process_expert_task's rows*(in/256)*2 (engine.c:929-942).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "main.h"
#include "math_dispatch.h"
#include "threadpool.h"

static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static int g_pool_threads;

static void ref_init_once(void)
{
	silu_table_init();
	math_dispatch_init();
	thread_pool = thread_pool_create(g_pool_threads);
}

static int ref_init(int nthreads)
{
	if (g_pool_threads == 0)
		g_pool_threads = nthreads;
	pthread_once(&g_once, ref_init_once);
	return thread_pool ? thread_pool->num_threads : -1;
}

int ref_pool_threads(void)
{
	return thread_pool ? thread_pool->num_threads : 0;
}

int ref_silu_table(float *tab, int nthreads)
{
	if (ref_init(nthreads) < 0)
		return -1;
	memcpy(tab, silu_table, sizeof(float) * SILU_TABLE_SIZE);
	return 0;
}

/* TIE's own dispatch_rms_norm (math_dispatch.c:198) on one row */
int ref_rms_norm(const float *x, const float *w, int size, float eps, float *out, int nthreads)
{
	if (ref_init(nthreads) < 0)
		return -1;
	MemType xi = {.type = GGML_TYPE_F32, .data = (void *)x};
	MemType oi = {.type = GGML_TYPE_F32, .data = out};
	Tensor wt;
	memset(&wt, 0, sizeof(wt));
	wt.mem = (MemType){.type = GGML_TYPE_F32, .data = (void *)w};
	dispatch_rms_norm(&xi, &wt, &oi, size, eps);
	return 0;
}

/* TIE's own dispatch_apply_residual (math_dispatch.c:468): acc += residual */
int ref_apply_residual(float *acc, const float *residual, int size, int nthreads)
{
	if (ref_init(nthreads) < 0)
		return -1;
	MemType a = {.type = GGML_TYPE_F32, .data = acc};
	MemType r = {.type = GGML_TYPE_F32, .data = (void *)residual};
	dispatch_apply_residual(&a, &r, size);
	return 0;
}

static size_t row_bytes(int type, int in_dim)
{
	switch (type) {
	case GGML_TYPE_F32:
		return (size_t)in_dim * 4;
	case GGML_TYPE_BF16:
		return (size_t)in_dim * 2;
	default:
		return (size_t)(in_dim / QK_K) * ggml_block_size(type);
	}
}

/* process_expert_task with byte-exact expert offsets (used only for BF16
 * experts when literal_bf16_stride == 0). */
static void expert_task_exact_stride(void *arg)
{
	expert_task_t *task = (expert_task_t *)arg;
	struct TIEContext *ctx = task->ctx;
	LayerWeights *l = &ctx->model->layers[task->layer_idx];
	int d = ctx->model->embed_dim, F = ctx->model->expert_ffn_dim;
	size_t gu = (size_t)task->expert_idx * F * row_bytes(l->ffn_up_exps.mem.type, d);
	size_t dn = (size_t)task->expert_idx * d * row_bytes(l->ffn_down_exps.mem.type, F);
	Tensor eg = {.mem.type = l->ffn_gate_exps.mem.type, .mem.data = (uint8_t *)l->ffn_gate_exps.mem.data + gu};
	Tensor eu = {.mem.type = l->ffn_up_exps.mem.type, .mem.data = (uint8_t *)l->ffn_up_exps.mem.data + gu};
	Tensor ed = {.mem.type = l->ffn_down_exps.mem.type, .mem.data = (uint8_t *)l->ffn_down_exps.mem.data + dn};
	MemType *h1 = &ctx->mem.ffn_hidden1_scratch[task->thread_id];
	MemType *h2 = &ctx->mem.ffn_hidden2_scratch[task->thread_id];
	MemType *yo = &ctx->mem.expert_outputs[task->thread_id];
	dispatch_mat_vec(ctx, &task->normed_input, &eg, h1, d, F, false);
	dispatch_mat_vec(ctx, &task->normed_input, &eu, h2, d, F, false);
	dispatch_swiglu_activation(h1, h2, F);
	dispatch_mat_vec(ctx, h1, &ed, yo, F, d, false);
}

int ref_moe_block(const float *x, int T, int d, int F, int E, int k, const float *router_w, const float *router_bias,
		  int routing, const float *probs_bias, const void *gate_w, int gate_type, const void *up_w, int up_type, const void *down_w, int down_type,
		  int literal_bf16_stride, float *out, int32_t *topk_idx, float *topk_w, float *logits_out,
		  int nthreads)
{
	if (nthreads < k)
		nthreads = k; /* tasks[num_threads] is indexed by j < k (model_qwen3.c:413,447) */
	if (ref_init(nthreads) < 0 || thread_pool->num_threads < k)
		return -1;

	Model model;
	memset(&model, 0, sizeof(model));
	LayerWeights layer;
	memset(&layer, 0, sizeof(layer));
	model.embed_dim = d;
	model.expert_count = E;
	model.expert_used_count = k;
	model.expert_ffn_dim = F;
	model.is_moe = 1;
	model.layers = &layer;
	layer.ffn_gate_inp.mem = (MemType){.type = GGML_TYPE_F32, .data = (void *)router_w};
	layer.ffn_gate_exps.mem = (MemType){.type = gate_type, .data = (void *)gate_w};
	layer.ffn_up_exps.mem = (MemType){.type = up_type, .data = (void *)up_w};
	layer.ffn_down_exps.mem = (MemType){.type = down_type, .data = (void *)down_w};

	struct TIEContext *ctx = calloc(1, sizeof(*ctx));
	ctx->model = &model;
	/* MoE scratch as model.c:416-433 */
	alloc_memtype(&ctx->mem.expert_scores, GGML_TYPE_F32, E);
	alloc_memtype(&ctx->mem.expert_out_fp32, GGML_TYPE_F32, d);
	ctx->mem.ffn_hidden1_scratch = calloc(k, sizeof(MemType));
	ctx->mem.ffn_hidden2_scratch = calloc(k, sizeof(MemType));
	ctx->mem.expert_outputs = calloc(k, sizeof(MemType));
	for (int j = 0; j < k; j++) {
		alloc_memtype(&ctx->mem.ffn_hidden1_scratch[j], GGML_TYPE_F32, F);
		alloc_memtype(&ctx->mem.ffn_hidden2_scratch[j], GGML_TYPE_F32, F);
		alloc_memtype(&ctx->mem.expert_outputs[j], GGML_TYPE_F32, d);
	}
	MemType in_buf = {.type = GGML_TYPE_F32, .data = (void *)x};
	MemType out_buf = {.type = GGML_TYPE_F32, .data = out};

	task_func_t task_fn = process_expert_task;
	if (!literal_bf16_stride &&
	    (gate_type == GGML_TYPE_BF16 || up_type == GGML_TYPE_BF16 || down_type == GGML_TYPE_BF16))
		task_fn = expert_task_exact_stride;

	expert_task_t tasks[thread_pool->num_threads];
	for (int i = 0; i < T; i++) {
		MemType xi = mem_slice(&in_buf, (size_t)i * d);
		MemType oi = mem_slice(&out_buf, (size_t)i * d);
		float *acc = ctx->mem.expert_out_fp32.data;

		dispatch_mat_vec(ctx, &xi, &layer.ffn_gate_inp, &ctx->mem.expert_scores, d, E, false);
		float *scores = (float *)ctx->mem.expert_scores.data;
		if (router_bias)
			for (int e = 0; e < E; e++)
				scores[e] += router_bias[e];
		if (logits_out)
			memcpy(logits_out + (size_t)i * E, scores, sizeof(float) * E);

		ExpertChoice top[k];
		float gv[k];
		if (routing == 1) {
			/* model_lfm2.c:437-467 */
			for (int e = 0; e < E; e++)
				scores[e] = 1.0f / (1.0f + expf(-scores[e]));
			float selection_scores[E];
			if (probs_bias) {
				for (int e = 0; e < E; e++)
					selection_scores[e] = scores[e] + probs_bias[e];
			} else {
				memcpy(selection_scores, scores, E * sizeof(float));
			}
			find_top_k(selection_scores, E, k, top);
			float sum_weights = 0.0f;
			for (int j = 0; j < k; j++) {
				gv[j] = top[j].index >= 0 ? scores[top[j].index] : 0.0f;
				sum_weights += gv[j];
			}
			float inv_sum = 1.0f / (sum_weights + 1e-6f);
			for (int j = 0; j < k; j++)
				gv[j] *= inv_sum;
		} else {
			find_top_k(scores, E, k, top);
			for (int j = 0; j < k; j++)
				gv[j] = top[j].score;
			softmax(gv, k);
		}

		for (int j = 0; j < k; j++) {
			tasks[j] = (expert_task_t){
				.ctx = ctx, .thread_id = j, .layer_idx = 0, .expert_idx = top[j].index, .normed_input = xi};
			thread_pool_submit(thread_pool, task_fn, &tasks[j]);
		}
		thread_pool_wait(thread_pool);

		memset(acc, 0, sizeof(float) * d);
		for (int j = 0; j < k; j++) {
			float gj = gv[j];
			float *yj = ctx->mem.expert_outputs[j].data;
			for (int c = 0; c < d; c++)
				acc[c] += gj * yj[c];
		}
		dispatch_convert(&ctx->mem.expert_out_fp32, &oi, d);

		if (topk_idx)
			for (int j = 0; j < k; j++)
				topk_idx[(size_t)i * k + j] = top[j].index;
		if (topk_w)
			memcpy(topk_w + (size_t)i * k, gv, sizeof(float) * k);
	}

	for (int j = 0; j < k; j++) {
		free_memtype(&ctx->mem.ffn_hidden1_scratch[j]);
		free_memtype(&ctx->mem.ffn_hidden2_scratch[j]);
		free_memtype(&ctx->mem.expert_outputs[j]);
	}
	free(ctx->mem.ffn_hidden1_scratch);
	free(ctx->mem.ffn_hidden2_scratch);
	free(ctx->mem.expert_outputs);
	free_memtype(&ctx->mem.expert_scores);
	free_memtype(&ctx->mem.expert_out_fp32);
	free(ctx);
	return 0;
}

/* ---- TIE's GGUF reader on a file (gguf_model_parse, gguf.c:977-1047, with
 * gguf_model_metadata_read, gguf.c:793, and gguf_model_map_weights,
 * gguf.c:892-966), for checking the library's own reader against it. */
void *ref_gguf_open(const char *path)
{
	char p[4096];
	strncpy(p, path, sizeof p - 1);
	p[sizeof p - 1] = 0;
	return gguf_model_parse(p);
}

void ref_gguf_close(void *h)
{
	if (h) {
		gguf_model_close((struct GGUFModel *)h);
		free(h);
	}
}

/* tensor count, data section offset and architecture id (detect_architecture) */
int ref_gguf_info(void *h, uint64_t *count, uint64_t *data_offset, int *arch)
{
	struct GGUFModel *g = (struct GGUFModel *)h;
	*count = g->tensor_count;
	*data_offset = g->tensor_data_offset;
	*arch = g->arch;
	return 0;
}

/* tensor i: name, type, dims, data pointer as a file offset, size */
int ref_gguf_tensor(void *h, uint64_t i, char *name, size_t cap, uint32_t *type, uint32_t *n_dims, uint64_t *ne,
		    uint64_t *file_offset, uint64_t *bytes)
{
	struct GGUFModel *g = (struct GGUFModel *)h;
	if (i >= g->tensor_count)
		return -1;
	const GGUFTensor *t = &g->tensors[i];
	strncpy(name, t->name, cap - 1);
	name[cap - 1] = 0;
	*type = t->type;
	*n_dims = t->n_dims;
	for (int j = 0; j < 4; j++)
		ne[j] = t->dimensions[j];
	*file_offset = (uint64_t)((uint8_t *)t->data - (uint8_t *)g->mapped_data);
	*bytes = t->size;
	return 0;
}

/* a scalar metadata value, its bytes as TIE's gguf_metadata_get_value copies them */
int ref_gguf_value(void *h, const char *key, void *value)
{
	char k[512];
	strncpy(k, key, sizeof k - 1);
	k[sizeof k - 1] = 0;
	return gguf_metadata_get_value((struct GGUFModel *)h, k, value);
}
