// capi.cpp -- the C ABI (include/tie_hip.h): device state, weight upload
// and cache, workspace, and the forward orchestration.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <string>
#include <mutex>
#include <stdlib.h>
#include <string.h>
#include <tuple>
#include <vector>

#include "common.h"
#include "gguf.h"

namespace tie {
int set_error(int code, const char *fmt, ...);
void clear_error();
int silu_table_host(float *tab, int n);
int rsqrt_table_host(std::vector<uint32_t> &tab, int &nbits);
double weight_mean_square(int type, const uint8_t *b, size_t n_bytes);
void f16_shifts(double ms_gate, double ms_down, int d, int F, int &h_shift, int &y_shift);
} // namespace tie

struct tie_hip_layer {
	tie::Layer L;
};

struct tie_hip_model {
	tie_hip_model_info info;
	std::vector<tie_hip_layer *> layers; // [n_layers], NULL for dense layers
	std::vector<float *> norms;          // [n_layers] device ffn_norm
};

struct tie_hip_matrix {
	tie::ExpertTensor W; // quantised / BF16 weights in the panel layout
	tie::Layer F;        // F32 weights: the router kernels' [rows][in] matrix
	void *alloc = nullptr;
	size_t bytes = 0;
};

namespace tie {

struct Ctx {
	int device = -1;
	hipStream_t stream = nullptr;
	float *silu = nullptr;
	// per-forward scratch, one per stream that forwards were enqueued on:
	// forwards on different streams never share a buffer
	std::map<hipStream_t, Workspace> ws;
	// host-pointer API: cached layers and staging buffers
	std::map<std::tuple<const void *, const void *, const void *, const void *, int, int, int, int, int, int, int,
			    const void *>,
		 tie_hip_layer *>
		cache;
	float *x_dev = nullptr, *out_dev = nullptr, *w_dev = nullptr;
	int32_t *idx_dev = nullptr;
	float *norm_dev = nullptr; // [io_d] RMSNorm weights of the host-pointer residual call
	size_t io_tokens = 0, io_d = 0, io_k = 0;
	uint32_t *rsq = nullptr;   // host RSQRTSS table (built at the first residual call)
	int rsq_bits = 0;
	// TIE_HIP_PATH_AUTO: TIE's bit-exact kernels up to this many tokens,
	// the matrix cores above (measured faster from T = 22 on at the 30B
	// shape, graph-timed: T=20 0.1002 / 0.1043 ms, T=22 0.1072 / 0.1065 ms,
	// T=24 0.1115 / 0.1083 ms exact / MFMA)
	int exact_max_t = 14;
	int debug_stale = 0; // one-launch decode calls left whose waits are made to give up (debug hook)
	std::recursive_mutex mu;
};

static Ctx g;
static int g_fail_alloc = 0;

// ------------------------------------------------- the no-allocation entry
// tie_hip_moe_forward_noalloc's workspace: a file-scope device array (one
// per GPU, held until the process ends).  Host code uses only g_scratch,
// its device address from hipGetSymbolAddress at tie_hip_init; the array's
// name is not a device address on the host.
constexpr size_t SCRATCH_BYTES = (size_t)24 << 20;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];
static uint8_t *g_scratch = nullptr;

// ---------------------------------------------------------------- profiling
struct ProfRec {
	int name, section;
	hipEvent_t a, b;
};
static bool g_prof = false;
static std::vector<std::string> g_prof_names;
static std::vector<ProfRec> g_prof_recs;
static std::vector<hipEvent_t> g_prof_pool;
static int g_prof_open = -1;

static hipEvent_t prof_event()
{
	if (!g_prof_pool.empty()) {
		hipEvent_t e = g_prof_pool.back();
		g_prof_pool.pop_back();
		return e;
	}
	hipEvent_t e = nullptr;
	if (hipEventCreate(&e) != hipSuccess)
		return nullptr;
	return e;
}

static int g_prof_section = 0;

void prof_begin(const char *name, hipStream_t)
{
	if (!g_prof)
		return;
	int id = -1;
	for (size_t i = 0; i < g_prof_names.size(); i++)
		if (g_prof_names[i] == name)
			id = (int)i;
	if (id < 0) {
		id = (int)g_prof_names.size();
		g_prof_names.push_back(name);
	}
	g_prof_open = id;
	g_prof_section++;
}

bool prof_kernel_events(hipEvent_t *start, hipEvent_t *stop)
{
	if (!g_prof || g_prof_open < 0)
		return false;
	ProfRec r{g_prof_open, g_prof_section, prof_event(), prof_event()};
	if (!r.a || !r.b) {
		if (r.a)
			g_prof_pool.push_back(r.a);
		if (r.b)
			g_prof_pool.push_back(r.b);
		return false;
	}
	g_prof_recs.push_back(r);
	*start = r.a;
	*stop = r.b;
	return true;
}

void prof_end(hipStream_t)
{
	g_prof_open = -1;
}

static void prof_reset()
{
	for (auto &r : g_prof_recs) {
		if (r.a)
			g_prof_pool.push_back(r.a);
		if (r.b)
			g_prof_pool.push_back(r.b);
	}
	g_prof_recs.clear();
	g_prof_names.clear();
	g_prof_open = -1;
}

#define HIP_TRY(expr)                                                                                        \
	do {                                                                                                 \
		hipError_t e_ = (expr);                                                                      \
		if (e_ != hipSuccess)                                                                        \
			return set_error(TIE_HIP_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_));      \
	} while (0)

static int dev_malloc(void **p, size_t bytes, const char *what)
{
	*p = nullptr;
	if (g_fail_alloc > 0 && --g_fail_alloc == 0)
		return set_error(TIE_HIP_ENOMEM, "injected allocation failure (%s, %zu bytes)", what, bytes);
	if (bytes == 0)
		bytes = 256;
	hipError_t e = hipMalloc(p, bytes);
	if (e != hipSuccess) {
		*p = nullptr;
		(void)hipGetLastError();
		return set_error(TIE_HIP_ENOMEM, "hipMalloc(%zu) for %s failed: %s", bytes, what, hipGetErrorString(e));
	}
	return TIE_HIP_OK;
}

static size_t align256(size_t n)
{
	return (n + 255) & ~(size_t)255;
}

static bool expert_type_ok(int t)
{
	return t == TIE_GGML_Q4_K || t == TIE_GGML_Q6_K || t == TIE_GGML_BF16;
}

static size_t row_bytes(int type, int in)
{
	switch (type) {
	case TIE_GGML_F32:
		return (size_t)in * 4;
	case TIE_GGML_BF16:
		return (size_t)in * 2;
	case TIE_GGML_Q4_K:
		return (size_t)(in / QK) * Q4K_BYTES;
	case TIE_GGML_Q6_K:
		return (size_t)(in / QK) * Q6K_BYTES;
	}
	return 0;
}

static int check_shape(int d, int F, int E)
{
	if (d <= 0 || F <= 0 || E <= 0)
		return set_error(TIE_HIP_EINVAL, "bad shape d=%d F=%d E=%d", d, F, E);
	if (d % QK || F % QK)
		return set_error(TIE_HIP_EINVAL, "d=%d and F=%d must be multiples of 256", d, F);
	if (d > 64 * QK || F > 64 * QK)
		return set_error(TIE_HIP_EINVAL, "d=%d, F=%d above the supported 16384", d, F);
	if (E > MAX_E)
		return set_error(TIE_HIP_EINVAL, "E=%d above %d", E, MAX_E);
	return TIE_HIP_OK;
}

static int ensure_init()
{
	if (g.device < 0)
		return set_error(TIE_HIP_ENOINIT, "tie_hip_init() has not been called");
	HIP_TRY(hipSetDevice(g.device));
	return TIE_HIP_OK;
}

// The workspace layout for P pairs (and as many tokens at most), F, d and E
// at most: its size, and (b != null) the pointers of *w into b.
static size_t carve_workspace(uint8_t *b, size_t P, size_t FF, size_t DD, size_t EE, Workspace *w,
			      bool direct_h = true)
{
	const size_t Tcap = P; // tokens <= pairs since k >= 1
	size_t off = 0;
	auto take = [&](size_t bytes) {
		size_t o = off;
		off += align256(bytes);
		return o;
	};
	const size_t o_idx = take(P * 4), o_w = take(P * 4), o_off = take((EE + 1) * 4), o_pairs = take(P * 4),
		     o_act = take((EE + 1) * 4), o_logits = take(Tcap * EE * 4), o_h = take(2 * P * FF * 4),
		     o_hb = take(P * FF * 2), o_y = take(P * DD * 4), o_xb = take(Tcap * DD * 2),
		     o_hlo = take(P * FF * 2), o_xlo = take(Tcap * DD * 2), o_nm = take(Tcap * DD * 4);
	const size_t o_bc = take(EE * 4), o_mk = take(EE * (size_t)T4((int)Tcap)), o_bk = take(EE * T4((int)Tcap) * 4);
	const size_t o_fl = take(Tcap * 4), o_fx = take(Tcap * 4), o_fc = take(4);
	const size_t o_xs = take(Tcap * 2 * (DD / 32 + 1) * 2);
	// h by expert for decode-sized matrix-core batches (not in the
	// no-allocation entry point's scratch: that path groups h by position)
	const size_t o_hd = direct_h ? take(EE * MFMA_DIRECT_T * FF * 2) : 0;
	const size_t o_lg = take(ONE_LG_COPIES * one_copy_words(EE) * 8),
		     o_dn = take(ONE_H_COPIES * one_copy_words((size_t)MAX_K * FF) * 8), o_st = take(4);
	if (!b)
		return off;
	w->topk_idx = (int32_t *)(b + o_idx);
	w->topk_w = (float *)(b + o_w);
	w->offsets = (int32_t *)(b + o_off);
	w->pairs = (int32_t *)(b + o_pairs);
	w->active = (int32_t *)(b + o_act);
	w->logits = (float *)(b + o_logits);
	w->h = (float *)(b + o_h);
	w->hb = (uint16_t *)(b + o_hb);
	w->hd = direct_h ? (uint16_t *)(b + o_hd) : nullptr;
	w->y = (float *)(b + o_y);
	w->normed = (float *)(b + o_nm);
	w->xb = (uint16_t *)(b + o_xb);
	w->hlo = (uint16_t *)(b + o_hlo);
	w->xlo = (uint16_t *)(b + o_xlo);
	w->xsum = (uint16_t *)(b + o_xs);
	w->bucket_cnt = (int32_t *)(b + o_bc);
	w->sel = b + o_mk;
	w->bucket = (int32_t *)(b + o_bk);
	w->tok_flag = (int32_t *)(b + o_fl);
	w->fix_list = (int32_t *)(b + o_fx);
	w->fix_count = (int32_t *)(b + o_fc);
	w->one_lg = (unsigned long long *)(b + o_lg);
	w->one_h = (unsigned long long *)(b + o_dn);
	w->one_seq = 0;
	w->one_status = (int32_t *)(b + o_st);
	w->cap_pairs = P;
	w->cap_F = FF;
	w->cap_d = DD;
	w->cap_E = EE;
	return off;
}

// Grow stream s's workspace to hold T tokens; *out = that workspace.
static int ensure_workspace(hipStream_t s, int T, int k, int d, int F, int E, Workspace **out)
{
	Workspace &w = g.ws[s];
	*out = &w;
	const size_t pairs = (size_t)(T > 0 ? T : 1) * k;
	if (w.alloc && pairs <= w.cap_pairs && (size_t)F <= w.cap_F && (size_t)d <= w.cap_d && (size_t)E <= w.cap_E)
		return TIE_HIP_OK;
	const size_t P = pairs > w.cap_pairs ? pairs : w.cap_pairs;
	const size_t FF = (size_t)F > w.cap_F ? F : w.cap_F;
	const size_t DD = (size_t)d > w.cap_d ? d : w.cap_d;
	const size_t EE = (size_t)E > w.cap_E ? E : w.cap_E;
	const size_t bytes = carve_workspace(nullptr, P, FF, DD, EE, nullptr);
	void *mem = nullptr;
	int32_t status = 0; // a given-up wait not yet reported survives the growth
	if (w.alloc) {
		// work still queued on s (or, through events, on any stream the
		// caller chained to it) may read the old buffer: drain the device
		HIP_TRY(hipDeviceSynchronize());
		HIP_TRY(hipMemcpy(&status, w.one_status, 4, hipMemcpyDeviceToHost));
		HIP_TRY(hipFree(w.alloc));
		w = Workspace();
	}
	int rc = dev_malloc(&mem, bytes, "workspace");
	if (rc)
		return rc;
	carve_workspace((uint8_t *)mem, P, FF, DD, EE, &w);
	w.alloc = mem;
	// the one-launch decode's words start at sequence 0 (every call uses a
	// later one)
	HIP_TRY(hipMemset(w.one_lg, 0, ONE_LG_COPIES * one_copy_words(EE) * 8));
	HIP_TRY(hipMemset(w.one_h, 0, ONE_H_COPIES * one_copy_words((size_t)MAX_K * FF) * 8));
	HIP_TRY(hipMemcpy(w.one_status, &status, 4, hipMemcpyHostToDevice));
	return TIE_HIP_OK;
}

// The status word of stream s's workspace: TIE_HIP_EHIP (and the word
// cleared) when a one-launch decode wait gave up since the last check.
// Synchronises s.
static int take_stream_status(hipStream_t s)
{
	auto it = g.ws.find(s);
	if (it == g.ws.end() || !it->second.alloc)
		return TIE_HIP_OK;
	HIP_TRY(hipStreamSynchronize(s));
	int32_t st = 0;
	HIP_TRY(hipMemcpy(&st, it->second.one_status, 4, hipMemcpyDeviceToHost));
	if (!st)
		return TIE_HIP_OK;
	const int32_t zero = 0;
	HIP_TRY(hipMemcpy(it->second.one_status, &zero, 4, hipMemcpyHostToDevice));
	return set_error(TIE_HIP_EHIP, "one-token forward: a wait between workgroups gave up (the GPU did not run "
				       "them together); that call's outputs are NaN");
}

static void free_layer(tie_hip_layer *l)
{
	if (!l)
		return;
	if (l->L.alloc)
		(void)hipFree(l->L.alloc);
	delete l;
}

static int create_layer(const tie_hip_layer_desc *ds, tie_hip_layer **out)
{
	*out = nullptr;
	int rc = check_shape(ds->d, ds->F, ds->E);
	if (rc)
		return rc;
	if (ds->router_type != TIE_GGML_F32)
		return set_error(TIE_HIP_EINVAL, "router type %d unsupported (F32 only)", ds->router_type);
	if (!expert_type_ok(ds->gate_type) || !expert_type_ok(ds->up_type) || !expert_type_ok(ds->down_type))
		return set_error(TIE_HIP_EINVAL, "expert types %d/%d/%d unsupported (Q4_K, Q6_K, BF16)", ds->gate_type,
				 ds->up_type, ds->down_type);
	if (!ds->router_w || !ds->gate_exps || !ds->up_exps || !ds->down_exps)
		return set_error(TIE_HIP_EINVAL, "null weight pointer");
	if (ds->routing != TIE_HIP_ROUTE_SOFTMAX && ds->routing != TIE_HIP_ROUTE_SIGMOID)
		return set_error(TIE_HIP_EINVAL, "routing mode %d unknown", ds->routing);
	if (ds->probs_bias && ds->routing != TIE_HIP_ROUTE_SIGMOID)
		return set_error(TIE_HIP_EINVAL, "probs_bias needs TIE_HIP_ROUTE_SIGMOID");

	const int d = ds->d, F = ds->F, E = ds->E;
	tie_hip_layer *l = new tie_hip_layer();
	Layer &L = l->L;
	L.d = d;
	L.F = F;
	L.E = E;
	auto setup = [&](ExpertTensor &t, int type, int rows, int in) {
		t.type = type;
		t.rows = rows;
		t.in = in;
		t.nb = in / QK;
		t.rt = rows / PANEL_ROWS;
		t.expert_bytes = (size_t)rows * row_bytes(type, in);
	};
	setup(L.gate, ds->gate_type, F, d);
	setup(L.up, ds->up_type, F, d);
	setup(L.down, ds->down_type, d, F);
	const size_t b_router = align256((size_t)E * d * 4), b_bias = align256((size_t)E * 4);
	const size_t b_gate = align256(E * L.gate.expert_bytes), b_up = align256(E * L.up.expert_bytes),
		     b_down = align256(E * L.down.expert_bytes);
	// [router | router bias | selection bias | transposed router | gate | up | down]
	L.bytes = 2 * b_router + 2 * b_bias + b_gate + b_up + b_down;
	rc = dev_malloc(&L.alloc, L.bytes, "layer weights");
	if (rc) {
		delete l;
		return rc;
	}
	uint8_t *base = (uint8_t *)L.alloc;
	L.router = (const float *)base;
	L.bias = ds->router_bias ? (const float *)(base + b_router) : nullptr;
	L.routing = ds->routing;
	L.pbias = ds->probs_bias ? (const float *)(base + b_router + b_bias) : nullptr;
	L.routerT = (const float *)(base + b_router + 2 * b_bias);
	L.gate.data = base + 2 * b_router + 2 * b_bias;
	L.up.data = L.gate.data + b_gate;
	L.down.data = L.up.data + b_up;

	const hipMemcpyKind kind = ds->src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
	// device sources may still be written by work on the caller's streams,
	// which the library's (non-blocking) stream does not wait for
	hipError_t e = ds->src_on_device ? hipDeviceSynchronize() : hipSuccess;
	if (e == hipSuccess)
		e = hipMemcpyAsync((void *)L.router, ds->router_w, (size_t)E * d * 4, kind, g.stream);
	if (e == hipSuccess && ds->router_bias)
		e = hipMemcpyAsync((void *)L.bias, ds->router_bias, (size_t)E * 4, kind, g.stream);
	if (e == hipSuccess && ds->probs_bias)
		e = hipMemcpyAsync((void *)L.pbias, ds->probs_bias, (size_t)E * 4, kind, g.stream);
	if (e == hipSuccess)
		e = launch_router_transpose(L, g.stream);
	struct Src {
		const ExpertTensor *t;
		const void *p;
	} srcs[3] = {{&L.gate, ds->gate_exps}, {&L.up, ds->up_exps}, {&L.down, ds->down_exps}};
	void *tmp = nullptr;
	for (int i = 0; i < 3 && e == hipSuccess; i++) {
		const size_t n = (size_t)E * srcs[i].t->expert_bytes;
		const uint8_t *src = (const uint8_t *)srcs[i].p;
		if (!ds->src_on_device) {
			rc = dev_malloc(&tmp, n, "upload staging");
			if (rc)
				break;
			e = hipMemcpyAsync(tmp, srcs[i].p, n, hipMemcpyHostToDevice, g.stream);
			src = (const uint8_t *)tmp;
		}
		if (e == hipSuccess)
			e = launch_repack(*srcs[i].t, src, E, ds->literal_bf16_stride, g.stream);
		if (e == hipSuccess)
			e = hipStreamSynchronize(g.stream);
		if (tmp) {
			(void)hipFree(tmp);
			tmp = nullptr;
		}
	}
	if (e == hipSuccess && rc == 0)
		e = hipStreamSynchronize(g.stream);
	if (e == hipSuccess && rc == 0) {
		// the f16 scales of h and y from samples of the gate and down
		// weights: a run of super-blocks (BF16: 256-weight runs) from the
		// middle of each of up to 128 experts, E plain copies (host or
		// device source: unified addressing)
		auto sample_ms = [&](int type, const void *src, size_t expert_bytes, double &ms) {
			const size_t bb = type == TIE_GGML_Q4_K ? Q4K_BYTES : type == TIE_GGML_Q6_K ? Q6K_BYTES : 2 * QK;
			const size_t per = std::min<size_t>(expert_bytes / bb, 32); // blocks per expert
			const int nexp = E < 128 ? E : 128, estep = E / nexp;
			ms = 0.0;
			if (per == 0)
				return hipSuccess;
			std::vector<uint8_t> smp((size_t)nexp * per * bb);
			for (int i = 0; i < nexp; i++) {
				const size_t off = (size_t)(i * estep) * expert_bytes + (expert_bytes / bb / 2) * bb;
				const size_t n = std::min(per * bb, (size_t)E * expert_bytes - off);
				const hipError_t err = hipMemcpy(smp.data() + (size_t)i * per * bb, (const uint8_t *)src + off,
								 n, hipMemcpyDefault);
				if (err != hipSuccess)
					return err;
			}
			ms = weight_mean_square(type, smp.data(), smp.size());
			return hipSuccess;
		};
		double ms_g = 0.0, ms_d = 0.0;
		e = sample_ms(ds->gate_type, ds->gate_exps, L.gate.expert_bytes, ms_g);
		if (e == hipSuccess)
			e = sample_ms(ds->down_type, ds->down_exps, L.down.expert_bytes, ms_d);
		if (e == hipSuccess)
			f16_shifts(ms_g, ms_d, d, F, L.h_shift, L.y_shift);
	}
	if (rc || e != hipSuccess) {
		free_layer(l);
		if (rc)
			return rc;
		return set_error(TIE_HIP_EHIP, "layer upload failed: %s", hipGetErrorString(e));
	}
	*out = l;
	return TIE_HIP_OK;
}

static bool capturing(hipStream_t s)
{
	hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
	if (hipStreamIsCapturing(s, &st) != hipSuccess) {
		(void)hipGetLastError();
		return true; // unknown: take the path that works either way
	}
	return st != hipStreamCaptureStatusNone;
}

// The block on device pointers; res (optional) is added to the combine
// (out = res + block, the residual add after the FFN).
static int forward(tie_hip_layer *layer, const float *x, int T, int k, float *out, int32_t *idx_out,
		   float *w_out, int flags, hipStream_t s, const float *res = nullptr, Workspace *preset = nullptr)
{
	if (!layer)
		return set_error(TIE_HIP_EINVAL, "null layer");
	const Layer &L = layer->L;
	if (T < 0)
		return set_error(TIE_HIP_EINVAL, "T=%d < 0", T);
	if (k < 1 || k > L.E || k > MAX_K)
		return set_error(TIE_HIP_EINVAL, "k=%d outside [1, min(E=%d, %d)]", k, L.E, MAX_K);
	if (T == 0)
		return TIE_HIP_OK;
	if (!x || !out)
		return set_error(TIE_HIP_EINVAL, "null x/out");
	const bool mfma = (flags & TIE_HIP_PATH_MFMA) || (!(flags & TIE_HIP_PATH_EXACT) && T > g.exact_max_t);
	if (mfma && !recompute_supported(L, k) && mfma_f16_operands(L))
		return set_error(TIE_HIP_EINVAL, "the MFMA path needs the exact per-token kernels for its range guard "
						 "(k * F too large for them: use TIE_HIP_PATH_EXACT)");
	if (mfma && L.gate.type != L.up.type)
		return set_error(TIE_HIP_EINVAL, "the MFMA path needs gate and up of one type (got %d, %d)", L.gate.type,
				 L.up.type);
	if (mfma && L.gate.type != TIE_GGML_BF16 && L.down.type == TIE_GGML_BF16)
		return set_error(TIE_HIP_EINVAL, "the MFMA path needs a quantised down when gate/up are quantised");
	Workspace *wsp = preset;
	int rc = preset ? TIE_HIP_OK : ensure_workspace(s, T, k, L.d, L.F, L.E, &wsp);
	if (rc)
		return rc;
	Workspace &ws = *wsp;
	if (mfma) {
		// logits (clearing the selection bytes or pair counts and the
		// recomputation count), then selection, pair lists (small T) or
		// selection bytes, and the A operand in one launch, then (large T)
		// the per-expert pair lists
		prof_begin("router", s);
		ZeroArgs z;
		if (route_appends(T)) {
			// the pair counts the routing appends to
			z.p = ws.bucket_cnt;
			z.n = L.E;
		} else {
			z.p2 = reinterpret_cast<int32_t *>(ws.sel);
			z.n2 = L.E * T4(T) / 4;
		}
		z.one = ws.fix_count;
		XConvArgs xc;
		const bool xconv = router_converts_x(L, T) && L.gate.type != TIE_GGML_BF16 && mfma_f16_operands(L);
		if (xconv) {
			// the tiled logits kernel writes the f16 A operand and range flags
			xc.xa = ws.xb;
			xc.flag = ws.tok_flag;
		}
		HIP_TRY(launch_router_logits(L, x, T, ws.logits, s, z, xc));
		HIP_TRY(launch_route_bucket(L, x, T, k, ws, s, xconv));
		prof_end(s);
		if (!route_appends(T)) {
			prof_begin("dispatch", s);
			HIP_TRY(launch_bucket_plan(L, T, k, ws, s));
			prof_end(s);
		}
		HIP_TRY(launch_mfma_experts(L, x, T, k, g.silu, ws, s));
		if (mfma_f16_operands(L) && combine_fix_preferred(L)) {
			// the combine of every token, except those whose activations
			// left the f16 range (listed by the kernels above; usually
			// none), which are recomputed exactly in the same launch, from
			// res as it was (res may be out)
			HIP_TRY(launch_combine_fix(L, x, k, g.silu, ws.topk_idx, ws.topk_w, ws.y, TIE_MFMA_Y16 != 0, L.y_shift,
						   out, res, ws.tok_flag, ws.fix_list, ws.fix_count, T, s));
		} else {
			// the same in two launches (the recomputation's LDS would cost
			// the combine occupancy); the combine skips the listed tokens
			prof_begin("combine", s);
			const bool y16 = TIE_MFMA_Y16 && mfma_f16_operands(L) && L.down.type != TIE_GGML_BF16;
			HIP_TRY(launch_combine(T, L.d, k, ws.topk_w, ws.topk_idx, ws.y, out, s, res,
					       mfma_f16_operands(L) ? ws.tok_flag : nullptr, y16, L.y_shift));
			prof_end(s);
			if (mfma_f16_operands(L))
				HIP_TRY(launch_recompute(L, x, k, g.silu, ws.topk_idx, ws.topk_w, out, res, ws.fix_list,
							 ws.fix_count, T, s));
		}
	} else if (T == 1 && !preset && !capturing(s) && decode_one_supported(L, k)) {
		// one token, one launch (eager calls on a workspace of their own:
		// the sequence number lives on the host, so a captured graph could
		// not advance it)
		if (++ws.one_seq == 0) {
			HIP_TRY(hipStreamSynchronize(s));
			HIP_TRY(hipMemset(ws.one_lg, 0, ONE_LG_COPIES * one_copy_words(ws.cap_E) * 8));
			HIP_TRY(hipMemset(ws.one_h, 0, ONE_H_COPIES * one_copy_words((size_t)MAX_K * ws.cap_F) * 8));
			ws.one_seq = 1;
		}
		uint32_t wseq = ws.one_seq;
		int spin = ONE_SPIN_MAX;
		if (g.debug_stale > 0) {
			// debug hook: wait for a stamp no workgroup writes, briefly
			g.debug_stale--;
			wseq ^= 0x80000000u;
			spin = 64;
		}
		HIP_TRY(launch_decode_one(L, x, k, g.silu, ws.topk_idx, ws.topk_w, out, res, ws.one_lg,
					  one_copy_words(ws.cap_E), ws.one_h, one_copy_words((size_t)MAX_K * ws.cap_F),
					  ws.one_seq, wseq, spin, ws.one_status, s));
	} else if (T == 1 && decode_supported(L, k)) {
		// one token: router logits, then the experts and the combine in two
		// launches (the selection runs in the gate/up prologue for E <= 128)
		prof_begin("router", s);
		HIP_TRY(launch_router_logits(L, x, 1, ws.logits, s));
		prof_end(s);
		const bool inl = L.E <= 128;
		if (!inl) {
			prof_begin("router_topk", s);
			HIP_TRY(launch_router_select(L, 1, k, ws.logits, ws.topk_idx, ws.topk_w, s));
			prof_end(s);
		}
		HIP_TRY(launch_decode(L, x, k, g.silu, ws.logits, ws.topk_idx, ws.topk_w, ws.h, out, res, nullptr, nullptr,
				      1, inl, false, s));
	} else {
		// routing, experts and the combine
		HIP_TRY(launch_exact_block(L, x, T, k, g.silu, ws, out, s, res));
	}
	if (idx_out)
		HIP_TRY(hipMemcpyAsync(idx_out, ws.topk_idx, (size_t)T * k * 4, hipMemcpyDeviceToDevice, s));
	if (w_out)
		HIP_TRY(hipMemcpyAsync(w_out, ws.topk_w, (size_t)T * k * 4, hipMemcpyDeviceToDevice, s));
	return TIE_HIP_OK;
}

// The host CPU's RSQRTSS table on the device (built once).
static int ensure_rsqrt()
{
	if (g.rsq)
		return TIE_HIP_OK;
	std::vector<uint32_t> tab;
	int nbits = 0;
	int rc = rsqrt_table_host(tab, nbits);
	if (rc)
		return rc;
	uint32_t *dev = nullptr;
	rc = dev_malloc((void **)&dev, tab.size() * 4, "rsqrt table");
	if (rc)
		return rc;
	HIP_TRY(hipMemcpy(dev, tab.data(), tab.size() * 4, hipMemcpyHostToDevice));
	g.rsq = dev;
	g.rsq_bits = nbits;
	return TIE_HIP_OK;
}

// out = hidden + block(rms_norm(hidden)): model_qwen3.c:392-401, 404-471,
// 491 (out may be hidden: TIE updates its hidden state in place).
static int forward_residual(tie_hip_layer *layer, const float *hidden, const float *norm_w, float eps, int T, int k,
			    float *out, int32_t *idx_out, float *w_out, int flags, hipStream_t s)
{
	if (!layer)
		return set_error(TIE_HIP_EINVAL, "null layer");
	const Layer &L = layer->L;
	if (T < 0)
		return set_error(TIE_HIP_EINVAL, "T=%d < 0", T);
	if (k < 1 || k > L.E || k > MAX_K)
		return set_error(TIE_HIP_EINVAL, "k=%d outside [1, min(E=%d, %d)]", k, L.E, MAX_K);
	if (T == 0)
		return TIE_HIP_OK;
	if (!hidden || !norm_w || !out)
		return set_error(TIE_HIP_EINVAL, "null hidden/ffn_norm/out");
	int rc = ensure_rsqrt();
	if (rc)
		return rc;
	Workspace *ws = nullptr;
	rc = ensure_workspace(s, T, k, L.d, L.F, L.E, &ws);
	if (rc)
		return rc;
	prof_begin("rmsnorm", s);
	HIP_TRY(launch_rmsnorm(hidden, norm_w, eps, T, L.d, ws->normed, g.rsq, g.rsq_bits, s));
	prof_end(s);
	return forward(layer, ws->normed, T, k, out, idx_out, w_out, flags, s, hidden);
}

} // namespace tie

using namespace tie;

extern "C" int tie_hip_init(int device)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	if (g.device >= 0) {
		if (g.device == device)
			return TIE_HIP_OK;
		return set_error(TIE_HIP_EINVAL, "already initialised on device %d", g.device);
	}
	int n = 0;
	HIP_TRY(hipGetDeviceCount(&n));
	if (device < 0 || device >= n)
		return set_error(TIE_HIP_EINVAL, "device %d not present (%d devices)", device, n);
	HIP_TRY(hipSetDevice(device));
	HIP_TRY(hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking));
	std::vector<float> tab(SILU_N);
	int rc = silu_table_host(tab.data(), SILU_N);
	if (rc)
		return rc;
	rc = dev_malloc((void **)&g.silu, SILU_N * sizeof(float), "silu table");
	if (rc)
		return rc;
	HIP_TRY(hipMemcpy(g.silu, tab.data(), SILU_N * sizeof(float), hipMemcpyHostToDevice));
	{
		void *p = nullptr;
		HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
		g_scratch = (uint8_t *)p;
	}
	g.device = device;
	return TIE_HIP_OK;
}

extern "C" void tie_hip_shutdown(void)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	if (g.device < 0)
		return;
	(void)hipSetDevice(g.device);
	(void)hipDeviceSynchronize();
	for (auto &kv : g.cache)
		free_layer(kv.second);
	g.cache.clear();
	for (auto &kv : g.ws)
		if (kv.second.alloc)
			(void)hipFree(kv.second.alloc);
	g.ws.clear();
	for (void *p : {(void *)g.x_dev, (void *)g.out_dev, (void *)g.w_dev, (void *)g.idx_dev, (void *)g.silu,
			(void *)g.norm_dev, (void *)g.rsq})
		if (p)
			(void)hipFree(p);
	g.x_dev = g.out_dev = g.w_dev = g.norm_dev = nullptr;
	g.idx_dev = nullptr;
	g.silu = nullptr;
	g.rsq = nullptr;
	g.rsq_bits = 0;
	g.io_tokens = g.io_d = g.io_k = 0;
	(void)hipStreamDestroy(g.stream);
	g.stream = nullptr;
	g.device = -1;
	g_scratch = nullptr;
}

extern "C" int tie_hip_set_silu_table(const float *table, int n)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	if (!table || n != SILU_N)
		return set_error(TIE_HIP_EINVAL, "silu table needs %d entries", SILU_N);
	HIP_TRY(hipStreamSynchronize(g.stream));
	HIP_TRY(hipMemcpy(g.silu, table, SILU_N * sizeof(float), hipMemcpyHostToDevice));
	return TIE_HIP_OK;
}

extern "C" int tie_hip_layer_create(const tie_hip_layer_desc *desc, tie_hip_layer **out)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	if (!out || !desc)
		return set_error(TIE_HIP_EINVAL, "null argument");
	*out = nullptr;
	int rc = ensure_init();
	if (rc)
		return rc;
	return create_layer(desc, out);
}

extern "C" void tie_hip_layer_destroy(tie_hip_layer *layer)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	if (!layer)
		return;
	if (g.device >= 0)
		(void)hipDeviceSynchronize(); // forwards on any stream may still read it
	free_layer(layer);
}

extern "C" size_t tie_hip_layer_bytes(const tie_hip_layer *layer)
{
	return layer ? layer->L.bytes : 0;
}

extern "C" int tie_hip_moe_forward(tie_hip_layer *layer, const float *x_dev, int T, int k, float *out_dev,
				   int32_t *topk_idx_dev, float *topk_w_dev, int flags, void *stream)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	hipStream_t s = stream ? (hipStream_t)stream : g.stream;
	return forward(layer, x_dev, T, k, out_dev, topk_idx_dev, topk_w_dev, flags, s);
}

extern "C" int tie_hip_moe_forward_noalloc(tie_hip_layer *layer, const float *x_dev, int T, int k, float *out_dev,
					   int32_t *topk_idx_dev, float *topk_w_dev, int flags, void *stream)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	if (!g_scratch)
		return set_error(TIE_HIP_ENOINIT, "scratch array address unknown (tie_hip_init failed)");
	if (!layer)
		return set_error(TIE_HIP_EINVAL, "null layer");
	const Layer &L = layer->L;
	if (T < 0 || k < 1 || k > L.E || k > MAX_K)
		return set_error(TIE_HIP_EINVAL, "bad T=%d or k=%d", T, k);
	const size_t P = (size_t)(T > 0 ? T : 1) * k;
	const size_t need = carve_workspace(nullptr, P, L.F, L.d, L.E, nullptr, false);
	if (need > SCRATCH_BYTES)
		return set_error(TIE_HIP_EINVAL,
				 "T=%d, k=%d needs %zu bytes of scratch, above the %zu of the no-allocation entry point "
				 "(use tie_hip_moe_forward)",
				 T, k, need, SCRATCH_BYTES);
	Workspace ws;
	carve_workspace(g_scratch, P, L.F, L.d, L.E, &ws, false);
	hipStream_t s = stream ? (hipStream_t)stream : g.stream;
	return forward(layer, x_dev, T, k, out_dev, topk_idx_dev, topk_w_dev, flags, s, nullptr, &ws);
}

// The host-buffer drop-ins: the layer comes from the weight cache (uploaded
// at the first call with these weights), x goes up, out and the selection
// come back, and the call returns after the stream has drained.
// With ffn_norm: the residual form, out = x + block(rms_norm(x)) (x and out
// may be the same buffer: TIE's hidden state).
static int moe_ffn_host(const float *x, int T, int d, int F, int E, int k, const void *router_w, int router_type,
			int routing, const float *probs_bias, const void *gate_exps, int gate_type, const void *up_exps,
			int up_type, const void *down_exps, int down_type, float *out, int32_t *topk_idx_opt,
			float *topk_w_opt, const float *ffn_norm = nullptr, float eps = 0.0f)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	rc = check_shape(d, F, E);
	if (rc)
		return rc;
	if (T < 0 || (T > 0 && (!x || !out)))
		return set_error(TIE_HIP_EINVAL, "bad T=%d or null x/out", T);
	auto key = std::make_tuple(router_w, gate_exps, up_exps, down_exps, router_type, gate_type, up_type, down_type,
				   d * 4096 + (F >> 8), E, routing, (const void *)probs_bias);
	tie_hip_layer *layer = nullptr;
	auto it = g.cache.find(key);
	if (it != g.cache.end()) {
		layer = it->second;
		if (layer->L.d != d || layer->L.F != F || layer->L.E != E)
			layer = nullptr;
	}
	if (!layer) {
		tie_hip_layer_desc ds;
		memset(&ds, 0, sizeof ds);
		ds.d = d;
		ds.F = F;
		ds.E = E;
		ds.router_w = router_w;
		ds.router_type = router_type;
		ds.gate_exps = gate_exps;
		ds.gate_type = gate_type;
		ds.up_exps = up_exps;
		ds.up_type = up_type;
		ds.down_exps = down_exps;
		ds.down_type = down_type;
		ds.routing = routing;
		ds.probs_bias = probs_bias;
		rc = create_layer(&ds, &layer);
		if (rc)
			return rc;
		g.cache[key] = layer;
	}
	if (T == 0)
		return TIE_HIP_OK;
	if (k < 1 || k > E || k > MAX_K)
		return set_error(TIE_HIP_EINVAL, "k=%d outside [1, min(E=%d, %d)]", k, E, MAX_K);
	if ((size_t)T > g.io_tokens || (size_t)d > g.io_d || (size_t)k > g.io_k) {
		HIP_TRY(hipStreamSynchronize(g.stream));
		for (void *p : {(void *)g.x_dev, (void *)g.out_dev, (void *)g.w_dev, (void *)g.idx_dev, (void *)g.norm_dev})
			if (p)
				(void)hipFree(p);
		g.x_dev = g.out_dev = g.w_dev = g.norm_dev = nullptr;
		g.idx_dev = nullptr;
		g.io_tokens = g.io_d = g.io_k = 0;
		const size_t nt = T, nd = d, nk = k;
		if ((rc = dev_malloc((void **)&g.x_dev, nt * nd * 4, "x staging")) ||
		    (rc = dev_malloc((void **)&g.out_dev, nt * nd * 4, "out staging")) ||
		    (rc = dev_malloc((void **)&g.w_dev, nt * nk * 4, "topk staging")) ||
		    (rc = dev_malloc((void **)&g.idx_dev, nt * nk * 4, "topk staging")) ||
		    (rc = dev_malloc((void **)&g.norm_dev, nd * 4, "ffn_norm staging")))
			return rc;
		g.io_tokens = nt;
		g.io_d = nd;
		g.io_k = nk;
	}
	HIP_TRY(hipMemcpyAsync(g.x_dev, x, (size_t)T * d * 4, hipMemcpyHostToDevice, g.stream));
	if (ffn_norm) {
		HIP_TRY(hipMemcpyAsync(g.norm_dev, ffn_norm, (size_t)d * 4, hipMemcpyHostToDevice, g.stream));
		rc = forward_residual(layer, g.x_dev, g.norm_dev, eps, T, k, g.x_dev, topk_idx_opt ? g.idx_dev : nullptr,
				      topk_w_opt ? g.w_dev : nullptr, TIE_HIP_PATH_AUTO, g.stream);
	} else {
		rc = forward(layer, g.x_dev, T, k, g.out_dev, topk_idx_opt ? g.idx_dev : nullptr,
			     topk_w_opt ? g.w_dev : nullptr, TIE_HIP_PATH_AUTO, g.stream);
	}
	if (rc)
		return rc;
	HIP_TRY(hipMemcpyAsync(out, ffn_norm ? g.x_dev : g.out_dev, (size_t)T * d * 4, hipMemcpyDeviceToHost, g.stream));
	if (topk_idx_opt)
		HIP_TRY(hipMemcpyAsync(topk_idx_opt, g.idx_dev, (size_t)T * k * 4, hipMemcpyDeviceToHost, g.stream));
	if (topk_w_opt)
		HIP_TRY(hipMemcpyAsync(topk_w_opt, g.w_dev, (size_t)T * k * 4, hipMemcpyDeviceToHost, g.stream));
	HIP_TRY(hipStreamSynchronize(g.stream));
	return take_stream_status(g.stream);
}

extern "C" void tie_hip_model_close(tie_hip_model *m)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	if (!m)
		return;
	if (g.device >= 0)
		(void)hipDeviceSynchronize(); // forwards on any stream may still read it
	for (auto *l : m->layers)
		free_layer(l);
	for (float *p : m->norms)
		if (p)
			(void)hipFree(p);
	delete m;
}

extern "C" int tie_hip_gguf_load(const char *path, tie_hip_model **out)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	if (!path || !out)
		return set_error(TIE_HIP_EINVAL, "null argument");
	*out = nullptr;
	int rc = ensure_init();
	if (rc)
		return rc;
	GGUFFile f;
	rc = f.open(path);
	if (rc)
		return rc;
	tie_hip_model *m = new tie_hip_model();
	rc = f.moe_info(m->info);
	if (rc) {
		delete m;
		return rc;
	}
	const tie_hip_model_info &I = m->info;
	m->layers.assign(I.n_layers, nullptr);
	m->norms.assign(I.n_layers, nullptr);
	auto fail = [&](int code) {
		tie_hip_model_close(m);
		return code;
	};
	auto dims = [](const GGUFTensor *t, uint64_t a, uint64_t b, uint64_t c) {
		return t->ne[0] == a && t->ne[1] == b && t->ne[2] == c && t->ne[3] == 1;
	};
	for (int n = I.first_moe_layer; n < I.n_layers; n++) {
		char name[96];
		auto get = [&](const char *what) {
			snprintf(name, sizeof name, "blk.%d.%s", n, what);
			return f.tensor(name);
		};
		const GGUFTensor *router = get("ffn_gate_inp.weight"), *gate = get("ffn_gate_exps.weight"),
				 *up = get("ffn_up_exps.weight"), *down = get("ffn_down_exps.weight"),
				 *norm = get("ffn_norm.weight"), *pbias = get("exp_probs_b.bias");
		if (!router || !gate || !up || !down)
			return fail(set_error(TIE_HIP_EINVAL, "layer %d: missing MoE FFN tensors", n));
		const uint64_t d = I.d, F = I.F, E = I.E;
		if (router->type != TIE_GGML_F32 || !dims(router, d, E, 1) || !dims(gate, d, F, E) || !dims(up, d, F, E) ||
		    !dims(down, F, d, E))
			return fail(set_error(TIE_HIP_EINVAL, "layer %d: MoE tensor shapes do not match d=%d F=%d E=%d", n,
					      I.d, I.F, I.E));
		if ((norm && (norm->type != TIE_GGML_F32 || !dims(norm, d, 1, 1))) ||
		    (pbias && (pbias->type != TIE_GGML_F32 || !dims(pbias, E, 1, 1))))
			return fail(set_error(TIE_HIP_EINVAL, "layer %d: ffn_norm / exp_probs_b shape or type", n));
		tie_hip_layer_desc ds;
		memset(&ds, 0, sizeof ds);
		ds.d = I.d;
		ds.F = I.F;
		ds.E = I.E;
		ds.router_w = router->data;
		ds.router_type = TIE_GGML_F32;
		ds.gate_exps = gate->data;
		ds.gate_type = gate->type;
		ds.up_exps = up->data;
		ds.up_type = up->type;
		ds.down_exps = down->data;
		ds.down_type = down->type;
		ds.routing = I.routing;
		ds.probs_bias = I.routing == TIE_HIP_ROUTE_SIGMOID && pbias ? (const float *)pbias->data : nullptr;
		rc = create_layer(&ds, &m->layers[n]);
		if (rc)
			return fail(rc);
		if (norm) {
			rc = dev_malloc((void **)&m->norms[n], d * 4, "ffn_norm");
			if (rc)
				return fail(rc);
			const hipError_t e = hipMemcpy(m->norms[n], norm->data, d * 4, hipMemcpyHostToDevice);
			if (e != hipSuccess)
				return fail(set_error(TIE_HIP_EHIP, "ffn_norm upload: %s", hipGetErrorString(e)));
		}
	}
	*out = m;
	return TIE_HIP_OK;
}

extern "C" void tie_hip_model_info_get(const tie_hip_model *m, tie_hip_model_info *info)
{
	if (m && info)
		*info = m->info;
}

extern "C" tie_hip_layer *tie_hip_model_layer(tie_hip_model *m, int n)
{
	return m && n >= 0 && n < (int)m->layers.size() ? m->layers[n] : nullptr;
}

extern "C" const float *tie_hip_model_ffn_norm(const tie_hip_model *m, int n)
{
	return m && n >= 0 && n < (int)m->norms.size() ? m->norms[n] : nullptr;
}

extern "C" int tie_hip_matrix_create(const void *w, int type, int rows, int in_dim, int src_on_device,
				     tie_hip_matrix **out)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	if (!out || !w)
		return set_error(TIE_HIP_EINVAL, "null argument");
	*out = nullptr;
	int rc = ensure_init();
	if (rc)
		return rc;
	if (rows <= 0 || in_dim <= 0 || rows % PANEL_ROWS)
		return set_error(TIE_HIP_EINVAL, "rows=%d must be a positive multiple of %d, in=%d", rows, PANEL_ROWS, in_dim);
	if (type != TIE_GGML_F32 && !expert_type_ok(type))
		return set_error(TIE_HIP_EINVAL, "matrix type %d unsupported (F32, Q4_K, Q6_K, BF16)", type);
	if (in_dim % QK || in_dim > 64 * QK)
		return set_error(TIE_HIP_EINVAL, "in=%d must be a multiple of 256 up to 16384", in_dim);
	tie_hip_matrix *m = new tie_hip_matrix();
	const size_t bytes = (size_t)rows * row_bytes(type, in_dim);
	rc = dev_malloc(&m->alloc, bytes, "matrix weights");
	if (rc) {
		delete m;
		return rc;
	}
	m->bytes = bytes;
	const hipMemcpyKind kind = src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
	// device sources may still be written by work on the caller's streams
	hipError_t e = src_on_device ? hipDeviceSynchronize() : hipSuccess;
	if (type == TIE_GGML_F32) {
		if (e == hipSuccess)
			e = hipMemcpyAsync(m->alloc, w, bytes, kind, g.stream);
		m->F.d = in_dim;
		m->F.E = rows;
		m->F.router = (const float *)m->alloc;
	} else {
		ExpertTensor &t = m->W;
		t.type = type;
		t.rows = rows;
		t.in = in_dim;
		t.nb = in_dim / QK;
		t.rt = rows / PANEL_ROWS;
		t.expert_bytes = bytes;
		t.data = (const uint8_t *)m->alloc;
		void *tmp = nullptr;
		const uint8_t *src = (const uint8_t *)w;
		if (!src_on_device) {
			rc = dev_malloc(&tmp, bytes, "upload staging");
			if (!rc && e == hipSuccess)
				e = hipMemcpyAsync(tmp, w, bytes, hipMemcpyHostToDevice, g.stream);
			src = (const uint8_t *)tmp;
		}
		if (!rc && e == hipSuccess)
			e = launch_repack(t, src, 1, 0, g.stream);
		if (e == hipSuccess)
			e = hipStreamSynchronize(g.stream);
		if (tmp)
			(void)hipFree(tmp);
	}
	if (e == hipSuccess && !rc)
		e = hipStreamSynchronize(g.stream);
	if (rc || e != hipSuccess) {
		(void)hipFree(m->alloc);
		delete m;
		if (rc)
			return rc;
		return set_error(TIE_HIP_EHIP, "matrix upload failed: %s", hipGetErrorString(e));
	}
	*out = m;
	return TIE_HIP_OK;
}

extern "C" void tie_hip_matrix_destroy(tie_hip_matrix *m)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	if (!m)
		return;
	if (g.device >= 0)
		(void)hipDeviceSynchronize(); // forwards on any stream may still read it
	if (m->alloc)
		(void)hipFree(m->alloc);
	delete m;
}

extern "C" int tie_hip_mat_mat(tie_hip_matrix *m, const float *x_dev, int T, float *out_dev, int flags, void *stream)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	if (!m)
		return set_error(TIE_HIP_EINVAL, "null matrix");
	if (T < 0)
		return set_error(TIE_HIP_EINVAL, "T=%d < 0", T);
	if (T == 0)
		return TIE_HIP_OK;
	if (!x_dev || !out_dev)
		return set_error(TIE_HIP_EINVAL, "null x/out");
	hipStream_t s = stream ? (hipStream_t)stream : g.stream;
	// the matrix cores only when asked for (Q4_K / Q6_K, rows a multiple of
	// 256): TIE_HIP_PATH_AUTO keeps TIE's exact row kernels at every T, so a
	// caller of dispatch_mat_mat gets TIE's bits unless it opts in
	const bool mfma_ok = !m->F.router && mfma_dense_supported(m->W, T);
	const bool mfma = (flags & TIE_HIP_PATH_MFMA) != 0;
	if (mfma && !mfma_ok)
		return set_error(TIE_HIP_EINVAL, "the matrix-core path needs a Q4_K / Q6_K matrix with rows a multiple of 256");
	prof_begin(mfma ? "dense_mfma" : "dense", s);
	if (mfma) {
		Workspace *ws = nullptr;
		rc = ensure_workspace(s, T, 1, m->W.in, QK, 1, &ws);
		if (rc)
			return rc;
		HIP_TRY(launch_mfma_dense(m->W, x_dev, T, out_dev, *ws, s));
	} else if (m->F.router) {
		HIP_TRY(launch_router_logits(m->F, x_dev, T, out_dev, s));
	} else if (dense_stream_supported(m->W, T)) {
		HIP_TRY(launch_dense_stream(m->W, x_dev, out_dev, s));
	} else if (dense_rows_supported(m->W, T)) {
		HIP_TRY(launch_dense_rows(m->W, x_dev, T, out_dev, s));
	} else {
		const int G = dense_groups(T);
		Workspace *ws = nullptr;
		rc = ensure_workspace(s, T, 1, m->W.in, QK, G, &ws);
		if (rc)
			return rc;
		HIP_TRY(launch_dense(m->W, x_dev, T, out_dev, *ws, s));
	}
	prof_end(s);
	return TIE_HIP_OK;
}

extern "C" int tie_hip_moe_forward_residual(tie_hip_layer *layer, const float *hidden_dev, const float *ffn_norm_dev,
					    float eps, int T, int k, float *out_dev, int32_t *topk_idx_dev, float *topk_w_dev,
					    int flags, void *stream)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	hipStream_t s = stream ? (hipStream_t)stream : g.stream;
	return forward_residual(layer, hidden_dev, ffn_norm_dev, eps, T, k, out_dev, topk_idx_dev, topk_w_dev, flags,
				s);
}

extern "C" int tie_hip_moe_ffn(const float *x, int T, int d, int F, int E, int k, const void *router_w,
			       int router_type, const void *gate_exps, int gate_type, const void *up_exps, int up_type,
			       const void *down_exps, int down_type, float *out, int32_t *topk_idx_opt,
			       float *topk_w_opt)
{
	return moe_ffn_host(x, T, d, F, E, k, router_w, router_type, TIE_HIP_ROUTE_SOFTMAX, nullptr, gate_exps,
			    gate_type, up_exps, up_type, down_exps, down_type, out, topk_idx_opt, topk_w_opt);
}

extern "C" int tie_hip_moe_ffn_lfm2(const float *x, int T, int d, int F, int E, int k, const void *router_w,
				    int router_type, const float *probs_bias_opt, const void *gate_exps, int gate_type,
				    const void *up_exps, int up_type, const void *down_exps, int down_type, float *out,
				    int32_t *topk_idx_opt, float *topk_w_opt)
{
	return moe_ffn_host(x, T, d, F, E, k, router_w, router_type, TIE_HIP_ROUTE_SIGMOID, probs_bias_opt,
			    gate_exps, gate_type, up_exps, up_type, down_exps, down_type, out, topk_idx_opt,
			    topk_w_opt);
}

extern "C" int tie_hip_qwen3_ffn(float *hidden, int T, int d, int F, int E, int k, const float *ffn_norm, float eps,
				 const void *router_w, int router_type, const void *gate_exps, int gate_type,
				 const void *up_exps, int up_type, const void *down_exps, int down_type,
				 int32_t *topk_idx_opt, float *topk_w_opt)
{
	if (!ffn_norm && T > 0)
		return set_error(TIE_HIP_EINVAL, "null ffn_norm");
	return moe_ffn_host(hidden, T, d, F, E, k, router_w, router_type, TIE_HIP_ROUTE_SOFTMAX, nullptr, gate_exps,
			    gate_type, up_exps, up_type, down_exps, down_type, hidden, topk_idx_opt, topk_w_opt, ffn_norm,
			    eps);
}

extern "C" int tie_hip_exact_max_tokens(void)
{
	return g.exact_max_t;
}

extern "C" void tie_hip_set_exact_max_tokens(int t)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	g.exact_max_t = t < 0 ? 0 : t;
}

extern "C" int tie_hip_stream_release(void *stream)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	auto it = g.ws.find(stream ? (hipStream_t)stream : g.stream);
	if (it == g.ws.end())
		return TIE_HIP_OK;
	HIP_TRY(hipDeviceSynchronize());
	if (it->second.alloc)
		HIP_TRY(hipFree(it->second.alloc));
	g.ws.erase(it);
	return TIE_HIP_OK;
}

extern "C" int tie_hip_stream_status(void *stream)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	return take_stream_status(stream ? (hipStream_t)stream : g.stream);
}

extern "C" void tie_hip_debug_decode_give_up(int n)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	g.debug_stale = n > 0 ? n : 0;
}

extern "C" int tie_hip_debug_layer_shifts(const tie_hip_layer *layer, int *h_shift, int *y_shift)
{
	if (!layer || !h_shift || !y_shift)
		return set_error(TIE_HIP_EINVAL, "null argument");
	*h_shift = layer->L.h_shift;
	*y_shift = layer->L.y_shift;
	return TIE_HIP_OK;
}

extern "C" void tie_hip_debug_fail_alloc(int n)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	g_fail_alloc = n < 0 ? 0 : n;
}

extern "C" int tie_hip_profile_enable(int on)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	prof_reset();
	g_prof = on != 0;
	return TIE_HIP_OK;
}

extern "C" int tie_hip_profile_read(char *names, size_t names_cap, double *total_ms, int *launches, int max_kernels)
{
	std::lock_guard<std::recursive_mutex> lk(g.mu);
	clear_error();
	int rc = ensure_init();
	if (rc)
		return rc;
	HIP_TRY(hipDeviceSynchronize());
	const int n = (int)g_prof_names.size() < max_kernels ? (int)g_prof_names.size() : max_kernels;
	std::string csv;
	for (int i = 0; i < n; i++) {
		total_ms[i] = 0.0;
		launches[i] = 0;
		csv += (i ? "," : "") + g_prof_names[i];
	}
	// a section's kernels are summed; launches counts sections
	int last_section = -1;
	for (auto &r : g_prof_recs) {
		if (r.name >= n)
			continue;
		float ms = 0.0f;
		if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
			total_ms[r.name] += ms;
			if (r.section != last_section)
				launches[r.name] += 1;
			last_section = r.section;
		}
	}
	if (names && names_cap) {
		strncpy(names, csv.c_str(), names_cap - 1);
		names[names_cap - 1] = 0;
	}
	return n;
}
