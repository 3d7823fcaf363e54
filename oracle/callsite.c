/* callsite.c -- TIE's MoE call sites, as INTEGRATION.md gives them, built
 * against TIE's own headers and run (TEST INFRASTRUCTURE ONLY).
 *
 * oracle/Makefile compiles this file with -I$(REF) (struct TIEContext,
 * Model, LayerWeights, Tensor, MemType: main.h, model.h:170-253,
 * engine.h:36-125), -DTIE_USE_HIP and TIE's warning flags plus -Werror,
 * with the call-site snippets that extract_callsite.py copies out of
 * INTEGRATION.md pasted into functions shaped like TIE's own:
 *
 *   qwen3_moe   the MoE branch of transformer_layer_qwen3 (model_qwen3.c:404-471)
 *   qwen3_ffn   its FFN half: RMSNorm, MoE, residual (model_qwen3.c:390-491)
 *   lfm2_moe    the MoE branch of transformer_layer_lfm2 (model_lfm2.c:414-497)
 *
 * and links it with libtie_hip.so and the reference build (oracle/_ref:
 * TIE's silu_table_init for the set-up snippet of engine_alloc,
 * engine.c:14-40).  It compiles only where the reference sources are; the
 * binary travels to the GPU box with the tree, where
 * tests/test_gpu_callsite.py runs it on seeded inputs and compares its
 * outputs with the oracle.
 *
 *   callsite DIR   reads DIR/meta.txt ("mode d F E k T gu_type down_type
 *                  eps"; mode 0 qwen3_moe, 1 qwen3_ffn, 2 lfm2_moe) and the
 *                  raw arrays DIR/{router,gate,up,down,x[,norm][,pbias]}.bin,
 *                  writes DIR/out.bin ([T][d] F32); exit status 0 on success.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "model.h"
#include "engine.h"
#include "main.h"
#include "tie_hip.h"

static int qwen3_moe(struct TIEContext *ctx, int layer_idx, int batch_len)
{
	LayerWeights *l = &ctx->model->layers[layer_idx];
#include "qwen3_moe.inc"
	return 0;
}

static int qwen3_ffn(struct TIEContext *ctx, int layer_idx, int batch_len)
{
	LayerWeights *l = &ctx->model->layers[layer_idx];
#include "qwen3_ffn.inc"
	return 0;
}

static int lfm2_moe(struct TIEContext *ctx, int layer_idx, int batch_len)
{
	LayerWeights *l = &ctx->model->layers[layer_idx];
	bool use_moe_ffn = ctx->model->is_moe && (layer_idx >= ctx->model->expert_leading_dense_layers);
#include "lfm2_moe.inc"
	return 0;
}

static void engine_setup(void)
{
	silu_table_init();
#include "init.inc"
}

static void *load(const char *dir, const char *name, size_t *bytes)
{
	char path[4096];
	snprintf(path, sizeof path, "%s/%s", dir, name);
	FILE *f = fopen(path, "rb");
	if (!f)
		return NULL;
	fseek(f, 0, SEEK_END);
	long n = ftell(f);
	fseek(f, 0, SEEK_SET);
	void *p = malloc(n > 0 ? (size_t)n : 1);
	if (p && n > 0 && fread(p, 1, (size_t)n, f) != (size_t)n) {
		free(p);
		p = NULL;
	}
	fclose(f);
	if (bytes)
		*bytes = (size_t)n;
	return p;
}

static void tensor(Tensor *t, void *data, size_t bytes, int type)
{
	t->mem.data = data;
	t->mem.n_bytes = bytes;
	t->mem.type = (GGMLType)type;
	t->size_in_bytes = bytes;
}

int main(int argc, char **argv)
{
	int mode, d, F, E, k, T, gu, dn;
	float eps;
	size_t nr, ng, nu, nd, nx, nn = 0, np = 0;
	if (argc != 2)
		return 2;
	const char *dir = argv[1];
	char path[4096];
	snprintf(path, sizeof path, "%s/meta.txt", dir);
	FILE *m = fopen(path, "r");
	if (!m || fscanf(m, "%d %d %d %d %d %d %d %d %f", &mode, &d, &F, &E, &k, &T, &gu, &dn, &eps) != 9)
		return 3;
	fclose(m);
	void *router = load(dir, "router.bin", &nr), *gate = load(dir, "gate.bin", &ng), *up = load(dir, "up.bin", &nu),
	     *down = load(dir, "down.bin", &nd);
	float *x = load(dir, "x.bin", &nx), *norm = load(dir, "norm.bin", &nn), *pbias = load(dir, "pbias.bin", &np);
	if (!router || !gate || !up || !down || !x || nx != (size_t)T * d * 4)
		return 4;

	/* what the call sites read of TIE's context: the model's shape, layer
	 * 0's tensors, the FFN buffers */
	Model *model = calloc(1, sizeof *model);
	LayerWeights *layers = calloc(1, sizeof *layers);
	struct TIEContext *ctx = calloc(1, sizeof *ctx);
	float *out = calloc((size_t)T * d, sizeof(float));
	model->embed_dim = d;
	model->expert_ffn_dim = F;
	model->expert_count = E;
	model->expert_used_count = k;
	model->is_moe = 1;
	model->norm_eps = eps;
	model->layers = layers;
	tensor(&layers[0].ffn_gate_inp, router, nr, GGML_TYPE_F32);
	tensor(&layers[0].ffn_gate_exps, gate, ng, gu);
	tensor(&layers[0].ffn_up_exps, up, nu, gu);
	tensor(&layers[0].ffn_down_exps, down, nd, dn);
	if (norm)
		tensor(&layers[0].ffn_norm, norm, nn, GGML_TYPE_F32);
	if (pbias && np)
		tensor(&layers[0].exp_probs_b_bias, pbias, np, GGML_TYPE_F32);
	ctx->model = model;
	ctx->mem.normed_ffn_input.data = x;
	ctx->mem.hidden_state.data = x;
	ctx->mem.ffn_down_output.data = out;

	engine_setup();
	int rc = mode == 0 ? qwen3_moe(ctx, 0, T) : mode == 1 ? qwen3_ffn(ctx, 0, T) : lfm2_moe(ctx, 0, T);
	tie_hip_shutdown(); /* model_language_cleanup */
	if (rc)
		return 5;
	snprintf(path, sizeof path, "%s/out.bin", dir);
	FILE *o = fopen(path, "wb");
	/* qwen3_ffn updates the hidden state in place */
	const float *res = mode == 1 ? x : out;
	if (!o || fwrite(res, sizeof(float), (size_t)T * d, o) != (size_t)T * d)
		return 6;
	fclose(o);
	printf("callsite mode %d T=%d d=%d: ok\n", mode, T, d);
	return 0;
}
