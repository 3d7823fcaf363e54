/*
 * tie_oracle.h -- CPU restatement of TIE's Qwen3-MoE FFN block.
 * TEST INFRASTRUCTURE ONLY (parity checker); see tie_oracle.c.
 */
#ifndef TIE_ORACLE_H
#define TIE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (gguf.h:8-36) */
enum { ORC_F32 = 0, ORC_Q4_K = 12, ORC_Q6_K = 14, ORC_BF16 = 30 };

#define ORC_SILU_N 8192 /* SILU_TABLE_SIZE, engine.h:10 */
#define ORC_MAX_K 32

float orc_fp16_to_fp32(uint16_t h);
void orc_q4k_scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *mn);
size_t orc_row_bytes(int type, int in_dim);

float orc_dot_f32(const float *x, const float *w, int n);
float orc_dot_bf16(const float *x, const uint16_t *w, int n);
float orc_dot_q4k_block(const float *x, const uint8_t *blk);
float orc_dot_q6k_block(const float *x, const uint8_t *blk);
int orc_matvec(const float *x, const void *W, int type, int in_dim, int rows, float *o);

int orc_silu_rcp_mode(void);
int orc_silu_table(float *tab, int mode);
void orc_swiglu(float *gate, const float *up, int n, const float *tab);

void orc_find_top_k(const float *logits, int E, int k, int32_t *idx, float *score);
void orc_softmax(float *v, int n);
void orc_sigmoid_route(const float *logits, int E, int k, const float *probs_bias, int32_t *idx, float *w);

int orc_moe_block(const float *x, int T, int d, int F, int E, int k, const float *router_w,
		  const float *router_bias, int routing, const float *probs_bias, const void *gate_w, int gate_type, const void *up_w, int up_type,
		  const void *down_w, int down_type, int literal_bf16_stride, const float *silu_tab, float *out,
		  int32_t *topk_idx, float *topk_w, float *logits_out, int nthreads);

void orc_rms_norm(const float *x, const float *w, int size, float eps, float *o);
int orc_qwen3_ffn(float *hidden, int T, int d, int F, int E, int k, const float *ffn_norm, float eps,
		  const float *router_w, const void *gate_w, int gate_type, const void *up_w, int up_type,
		  const void *down_w, int down_type, const float *silu_tab, int32_t *topk_idx, float *topk_w,
		  int nthreads);
void orc_dequant_q4k(const uint8_t *blocks, int n, float *y);
void orc_dequant_q6k(const uint8_t *blocks, int n, float *y);
void orc_expf_array(const float *in, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
