// Host runtime of the StrasGPT forward pass on one MI355X.
//
// Load: every tensor of the safetensors description is read once (pread
// into pinned staging buffers, two in flight) and copied to HBM; names are
// matched like the reference loader (source/transformer.c:513-625: the
// Hugging Face names and the Qwen3-VL "model.language_model." aliases),
// sizes are checked exactly, and missing tensors are an error. Q, K and V
// of a layer land in one fused [(qh + 2 kvh) hd][d] matrix.
//
// Predict: the reference's chunk loop (source/transformer.c:1607-1727)
// over at most 512 tokens. A single-token chunk runs the decode kernels
// (GEMV with fused RMSNorm and epilogues, split-K attention); longer
// chunks run the MFMA GEMMs and the tiled prefill attention. The cache
// position lives in device memory, so the single-token step can be
// captured once as a HIP graph and replayed by the greedy generation loop,
// whose argmax kernel feeds the next token and advances the position on
// the device.
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <vector>

#include "hip_check.h"
#include "kernels.h"
#include "runtime.h"
#include "sampler_impl.h"
#include "safetensors.h"

namespace {

enum WClass {
  W_EMB, W_MHA_NORM, W_Q, W_Q_NORM, W_K, W_K_NORM, W_V, W_O, W_FFN_NORM, W_GATE,
  W_UP, W_DOWN, W_OUT_NORM, W_OUT, W_ROUTER, W_GB, W_GS, W_UB, W_US, W_DB, W_DS,
  W_COUNT
};

const char* kClassName[W_COUNT] = {
    "embedding", "mha_norm", "mha_q", "mha_q_norm", "mha_k", "mha_k_norm", "mha_v",
    "mha_out", "ffn_norm", "ffn_fc", "ffn_up", "ffn_out", "out_norm", "out",
    "moe_router", "moe_gate_blocks", "moe_gate_scales", "moe_up_blocks",
    "moe_up_scales", "moe_down_blocks", "moe_down_scales"};

struct LayerName {
  const char* suffix;
  WClass cls;
};
const LayerName kLayerNames[] = {
    {"input_layernorm.weight", W_MHA_NORM},
    {"self_attn.q_proj.weight", W_Q},
    {"self_attn.q_norm.weight", W_Q_NORM},
    {"self_attn.k_proj.weight", W_K},
    {"self_attn.k_norm.weight", W_K_NORM},
    {"self_attn.v_proj.weight", W_V},
    {"self_attn.o_proj.weight", W_O},
    {"post_attention_layernorm.weight", W_FFN_NORM},
    {"mlp.gate_proj.weight", W_GATE},
    {"mlp.up_proj.weight", W_UP},
    {"mlp.down_proj.weight", W_DOWN},
    {"mlp.router.weight", W_ROUTER},
    {"mlp.experts.gate_proj_blocks", W_GB},
    {"mlp.experts.gate_proj_scales", W_GS},
    {"mlp.experts.up_proj_blocks", W_UB},
    {"mlp.experts.up_proj_scales", W_US},
    {"mlp.experts.down_proj_blocks", W_DB},
    {"mlp.experts.down_proj_scales", W_DS},
};

// Name -> (class, layer). Accepts the base names and the
// "model.language_model." aliases (reference source/transformer.c:520-574).
bool classify(const char* name, WClass* cls, long* layer) {
  char buf[SAFETENSORS_MAX_STRING];
  const char* alias = "model.language_model.";
  if (strncmp(name, alias, strlen(alias)) == 0) {
    snprintf(buf, sizeof(buf), "model.%s", name + strlen(alias));
    name = buf;
  }
  *layer = 0;
  if (strcmp(name, SAFETENSORS_PATTERN_EMBEDDING_WEIGHT) == 0) { *cls = W_EMB; return true; }
  if (strcmp(name, SAFETENSORS_PATTERN_OUT_NORM_WEIGHT) == 0) { *cls = W_OUT_NORM; return true; }
  if (strcmp(name, SAFETENSORS_PATTERN_OUT_WEIGHT) == 0) { *cls = W_OUT; return true; }
  const char* pre = "model.layers.";
  if (strncmp(name, pre, strlen(pre)) != 0) return false;
  const char* p = name + strlen(pre);
  if (*p < '0' || *p > '9') return false;
  long idx = 0;
  while (*p >= '0' && *p <= '9') idx = idx * 10 + (*p++ - '0');
  if (*p++ != '.') return false;
  for (const LayerName& ln : kLayerNames) {
    if (strcmp(p, ln.suffix) == 0) {
      *cls = ln.cls;
      *layer = idx;
      return true;
    }
  }
  return false;
}

bool is_global(int c) { return c == W_EMB || c == W_OUT_NORM || c == W_OUT; }

struct Summary {
  size_t bytes = 0;
  float first[3] = {0, 0, 0}, last[3] = {0, 0, 0};
  bool present = false;
};

double now_s() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

}  // namespace

struct transformer_device {
  hipStream_t stream = nullptr;
  int d = 0, hd = 0, H = 0, L = 0, qh = 0, kvh = 0, V = 0, ctx = 0, qd = 0, kvd = 0;
  int qkv_rows = 0, E = 0, topk = 0;
  float eps = 0.f;
  bool qk_norm = false, moe = false, tied = false;
  int pb = 0, po = 0, pst = 0;
  size_t per_layer[W_COUNT] = {0};  // bytes per layer (or total for globals)
  void* w[W_COUNT] = {nullptr};
  // activations [chunk][...]
  float *x = nullptr, *xn = nullptr, *q = nullptr, *att = nullptr, *act = nullptr;
  // prefill GEMM inputs as bf16 hi/lo planes, split-K partial sums
  uint16_t *xn_hi = nullptr, *xn_lo = nullptr, *att_hi = nullptr, *att_lo = nullptr;
  uint16_t *act_hi = nullptr, *act_lo = nullptr;
  float* ws = nullptr;
  int ws_splits = 0;
  size_t ws_rows = 0;   // split-K workspace: ws_splits x ws_rows rows of d
  size_t chunk = 0;     // prefill rows per forward_chunk (>= the API's 512)
  float *kraw = nullptr, *logits = nullptr;
  int logits_rows = 0;
  size_t host_pos = 0;  // host mirror of *pos (profiling byte counts)
  bool use_graph = true;  // STRASGPT_DECODE_GRAPH=0: eager decode steps
  int decode_mode = TRANSFORMER_DECODE_GRAPH;
  float *kc = nullptr, *vc = nullptr, *rope = nullptr;
  // KV-cache format: fp32 (the reference's) or bf16 (kv_bf16: 2-byte
  // elements in the same [L][kvh][ctx][hd] layout, values rounded to
  // nearest even); with bf16, prefill stages the raw keys in kstage
  // [chunk][kvd] fp32 until their norm and RoPE
  int kv_bf16 = 0;
  float* kstage = nullptr;
  // The cache rows as bf16 hi/lo planes, the operands of the attention
  // kernels: K [L][kvh][ctx][hd], V transposed [L][kvh][hd][ctx_pad];
  // zero-initialised; rows [0, cached_count) valid (every layer).
  uint16_t *kp_hi = nullptr, *kp_lo = nullptr, *vt_hi = nullptr, *vt_lo = nullptr;
  int ctx_pad = 0;
  int *tok = nullptr, *pos = nullptr, *next = nullptr, *seq = nullptr, *seq_len = nullptr;
  int seq_cap = 0;
  float* attn_part = nullptr;
  int attn_splits = 0;
  unsigned* attn_cnt = nullptr;  // [kvh] decode attention arrivals
  float* gemv_part = nullptr;    // [8][d] split-K GEMV partial sums (rows > 16384)
  unsigned* gemv_cnt = nullptr;  // [kGemvCounters] their arrival counters
  float* am_v = nullptr;
  int* am_i = nullptr;
  int* h_tok = nullptr;
  int* h_pos = nullptr;
  int* h_next = nullptr;
  hipGraphExec_t graph = nullptr;       // decode step + argmax
  hipGraphExec_t graph_body = nullptr;  // decode step alone (the sampled loop)
  int precision = sg::GEMM_SPLIT2;
  float* cap_out = nullptr;
  float* cap_final = nullptr;
  float* cap_dev = nullptr;
  float* cap_final_dev = nullptr;
  // MoE scratch
  int* moe_sel = nullptr;
  float* moe_w = nullptr;
  float* moe_act = nullptr;
  // MoE prefill: the grouped GEMMs' A rows in expert order, bf16 hi/lo
  uint16_t *moe_ahi = nullptr, *moe_alo = nullptr;
  float* moe_logits = nullptr;  // [E] router logits of a decode step
  int* moe_offs = nullptr;   // [E + 1] grouped prefill: slot ranges per expert
  int* moe_order = nullptr;  // [T * topk] slots sorted by expert
  float* moe_out = nullptr;  // [T * topk][d] per-slot down projections
  Summary summary[W_COUNT];
  // measurement hooks
  bool prof = false;
  struct Pending {
    int cls;
    hipEvent_t a, b;
    double bytes, flops;
  };
  std::vector<Pending> pending;
  std::vector<hipEvent_t> event_pool;
  transformer_kernel_stat_t stat[TRANSFORMER_K_CLASS_COUNT];
};

namespace {

typedef transformer_device Dev;

template <typename T>
T* dalloc(size_t count) {
  void* p = nullptr;
  if (count == 0) count = 1;
  HIP_CHECK(hipMalloc(&p, count * sizeof(T)));
  return (T*)p;
}

void drop_graphs(Dev* D) {
  if (D->graph) HIP_CHECK(hipGraphExecDestroy(D->graph));
  if (D->graph_body) HIP_CHECK(hipGraphExecDestroy(D->graph_body));
  D->graph = D->graph_body = nullptr;
}

// The K and V caches (`cache` elements each) in D's format, zeroed, and for
// a bf16 cache the prefill key staging rows.
void alloc_kv(Dev* D, size_t cache) {
  const size_t es = D->kv_bf16 ? 2 : 4;
  D->kc = (float*)dalloc<char>(cache * es);
  D->vc = (float*)dalloc<char>(cache * es);
  HIP_CHECK(hipMemsetAsync(D->kc, 0, cache * es, D->stream));
  HIP_CHECK(hipMemsetAsync(D->vc, 0, cache * es, D->stream));
  if (D->kv_bf16) D->kstage = dalloc<float>(D->chunk * D->kvd);
}

uint16_t* W16(Dev* D, int cls, int layer = 0) {
  return (uint16_t*)((char*)D->w[cls] + (size_t)layer * D->per_layer[cls]);
}
uint8_t* W8(Dev* D, int cls, int layer = 0) {
  return (uint8_t*)D->w[cls] + (size_t)layer * D->per_layer[cls];
}

// Brackets one launch with events when profiling is on.
struct Prof {
  Dev* D;
  int cls;
  double bytes, flops;
  hipEvent_t a = nullptr, b = nullptr;
  Prof(Dev* d, int c, double by, double fl) : D(d), cls(c), bytes(by), flops(fl) {
    if (!D->prof) return;
    a = take();
    b = take();
    HIP_CHECK(hipEventRecord(a, D->stream));
  }
  ~Prof() {
    if (!D->prof) return;
    HIP_CHECK(hipEventRecord(b, D->stream));
    D->pending.push_back({cls, a, b, bytes, flops});
  }
  hipEvent_t take() {
    if (D->event_pool.empty()) {
      hipEvent_t e;
      HIP_CHECK(hipEventCreate(&e));
      return e;
    }
    hipEvent_t e = D->event_pool.back();
    D->event_pool.pop_back();
    return e;
  }
};

// Called after a stream synchronisation: folds finished launches into the
// per-class statistics.
void harvest(Dev* D) {
  for (auto& p : D->pending) {
    float ms = 0.f;
    HIP_CHECK(hipEventElapsedTime(&ms, p.a, p.b));
    transformer_kernel_stat_t& st = D->stat[p.cls];
    st.launches++;
    st.total_ms += ms;
    st.bytes += p.bytes;
    st.flops += p.flops;
    D->event_pool.push_back(p.a);
    D->event_pool.push_back(p.b);
  }
  D->pending.clear();
}

// -------------------------------------------------------------- upload --

struct Stager {
  static constexpr size_t kChunk = 64u << 20;
  void* buf[2] = {nullptr, nullptr};
  hipEvent_t ev[2];
  bool used[2] = {false, false};
  int cur = 0;
  hipStream_t s;
  explicit Stager(hipStream_t st) : s(st) {
    for (int i = 0; i < 2; i++) {
      HIP_CHECK(hipHostMalloc(&buf[i], kChunk, hipHostMallocDefault));
      HIP_CHECK(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
    }
  }
  ~Stager() {
    HIP_CHECK(hipStreamSynchronize(s));
    for (int i = 0; i < 2; i++) {
      HIP_CHECK(hipHostFree(buf[i]));
      HIP_CHECK(hipEventDestroy(ev[i]));
    }
  }
  void copy(int fd, size_t offset, size_t size, void* dst) {
    size_t done = 0;
    while (done < size) {
      const size_t n = size - done < kChunk ? size - done : kChunk;
      if (used[cur]) HIP_CHECK(hipEventSynchronize(ev[cur]));
      size_t got = 0;
      while (got < n) {
        ssize_t r = pread(fd, (char*)buf[cur] + got, n - got, (off_t)(offset + done + got));
        if (r <= 0) ST_DIE("failed to read from file");
        got += (size_t)r;
      }
      HIP_CHECK(hipMemcpyAsync((char*)dst + done, buf[cur], n, hipMemcpyHostToDevice, s));
      HIP_CHECK(hipEventRecord(ev[cur], s));
      used[cur] = true;
      cur ^= 1;
      done += n;
    }
  }
};

void build_rope_table(const transformer_configuration_t* c, std::vector<float>& t) {
  // Reference state_from_safetensors (source/transformer.c:126-146), same
  // fp32 libm calls so the table is bit-identical to the CPU path's.
  const size_t hd = c->head_dim;
  const bool interleaved = c->rope_pair_stride == 2;
  const float coef = interleaved ? 1.0f : 2.0f;
  t.assign(c->context_len * hd, 0.0f);
  for (size_t i = 0; i < c->context_len; i++) {
    for (size_t j = 0; j < c->rope_pair_bound; j += c->rope_pair_stride) {
      float freq = 1.0f / powf(c->rope_theta, (coef * (float)j) / (float)hd);
      float val = (float)i * freq;
      t[i * hd + j] = cosf(val);
      t[i * hd + j + c->rope_pair_offset] = sinf(val);
    }
  }
}

bool has_tensor(const safetensors_t* s, WClass want) {
  for (size_t i = 0; i < s->tensor_count; i++) {
    WClass c;
    long l;
    if (classify(s->tensor[i].name, &c, &l) && c == want) return true;
  }
  return false;
}

// ------------------------------------------------------------- forward --

enum {
  K_QKV_GEMV = TRANSFORMER_K_QKV_GEMV, K_ATT_DEC = TRANSFORMER_K_ATTENTION_DECODE,
  K_O_GEMV = TRANSFORMER_K_O_GEMV, K_GU_GEMV = TRANSFORMER_K_GATE_UP_GEMV,
  K_DOWN_GEMV = TRANSFORMER_K_DOWN_GEMV, K_LOGITS = TRANSFORMER_K_LOGITS_GEMV,
  K_ARGMAX = TRANSFORMER_K_ARGMAX, K_ROUTE = TRANSFORMER_K_MOE_ROUTE,
  K_MOE_GU = TRANSFORMER_K_MOE_GATE_UP, K_MOE_DOWN = TRANSFORMER_K_MOE_DOWN,
  K_QKV_GEMM = TRANSFORMER_K_QKV_GEMM, K_ATT_PRE = TRANSFORMER_K_ATTENTION_PREFILL,
  K_O_GEMM = TRANSFORMER_K_O_GEMM, K_GU_GEMM = TRANSFORMER_K_GATE_UP_GEMM,
  K_DOWN_GEMM = TRANSFORMER_K_DOWN_GEMM, K_ELEM = TRANSFORMER_K_ELEMENTWISE,
  K_ROUTE_PRE = TRANSFORMER_K_MOE_ROUTE_PREFILL, K_MOE_GU_PRE = TRANSFORMER_K_MOE_GATE_UP_PREFILL,
  K_MOE_DOWN_PRE = TRANSFORMER_K_MOE_DOWN_PREFILL
};

double mxfp4_bytes(double values) { return values * (0.5 + 1.0 / 32.0); }

// From this many tokens the MoE FFN runs as grouped GEMMs (below: GEMVs
// per token and slot).
constexpr int kMoeGroupedMinTokens = 8;

// MoE FFN of T rows: RMSNorm, router top-k, MXFP4 SwiGLU experts, routed
// down-projection accumulated into the residual stream.
// Returns true when the routed sum of the expert outputs is left for the
// next prefill_norm to add (D->moe_out, weights D->moe_w).
bool ffn_moe(Dev* D, int l, int T) {
  hipStream_t s = D->stream;
  const double d = D->d, H = D->H, k = D->topk;
  const bool fused = T == 1 && sg::moe_route_logits_supported(D->E, D->topk, D->d);
  if (fused) {
    // decode: RMSNorm + router logits in one launch; the expert kernels
    // select the top-k from the logits themselves
    Prof pr(D, K_ROUTE, (double)D->E * d * 2, 2.0 * D->E * d);
    sg::moe_route_logits(D->x, W16(D, W_FFN_NORM, l), D->eps, W16(D, W_ROUTER, l), D->E, D->d, D->moe_logits,
                         D->xn, s);
  } else {
    if (T == 1) {  // (prefill: the RMSNorm rows came with the residual add)
      Prof pr(D, K_ELEM, 2.0 * T * d * 4, 0);
      sg::rmsnorm_rows(D->x, W16(D, W_FFN_NORM, l), D->xn, T, D->d, D->eps, s);
    }
    {
      Prof pr(D, T == 1 ? K_ROUTE : K_ROUTE_PRE, (double)D->E * d * 2, 2.0 * T * D->E * d);
      sg::moe_route(D->xn, T, W16(D, W_ROUTER, l), D->E, D->d, D->topk, D->moe_sel, D->moe_w, s);
    }
  }
  if (T >= kMoeGroupedMinTokens) {
    // prefill: slots grouped by expert, each expert's weights read once per
    // 32-slot tile (MFMA GEMMs), then the routed sum in top-k order
    const int n = T * D->topk;
    const double used = std::min((double)n, (double)D->E);
    sg::moe_group(D->moe_sel, n, D->E, D->moe_offs, D->moe_order, s);
    sg::MoeGemmParams g{};
    g.blocks = W8(D, W_GB, l);
    g.scales = W8(D, W_GS, l);
    g.blocks2 = W8(D, W_UB, l);
    g.scales2 = W8(D, W_US, l);
    g.a = D->xn;
    g.a_per_token = 1;
    g.offs = D->moe_offs;
    g.order = D->moe_order;
    g.slots = n;
    g.topk = D->topk;
    g.E = D->E;
    g.N = D->H;
    g.K = D->d;
    g.y = D->moe_act;
    // A: the RMSNorm rows' planes, one per token, read through the grouping
    g.a_hi = D->xn_hi;
    g.a_lo = D->xn_lo;
    if (!sg::moe_group_gemm2_ok(g)) g.a_hi = g.a_lo = nullptr;
    sg::MoeGemmParams dn{};
    dn.blocks = W8(D, W_DB, l);
    dn.scales = W8(D, W_DS, l);
    dn.a = D->moe_act;
    dn.a_per_token = 0;
    dn.offs = D->moe_offs;
    dn.order = D->moe_order;
    dn.slots = n;
    dn.topk = D->topk;
    dn.E = D->E;
    dn.N = D->d;
    dn.K = D->H;
    dn.y = D->moe_out;
    dn.a_hi = D->moe_ahi;
    dn.a_lo = D->moe_alo;
    if (!sg::moe_group_gemm2_ok(dn)) dn.a_hi = dn.a_lo = nullptr;
    // the gate/up GEMM writes the down GEMM's A planes in expert order
    // when both run the pipelined kernel (no gather between them)
    const bool planes = g.a_hi && dn.a_hi;
    if (planes) {
      g.y_hi = D->moe_ahi;
      g.y_lo = D->moe_alo;
    }
    {
      Prof pr(D, K_MOE_GU_PRE, used * mxfp4_bytes(2 * H * d), 4.0 * n * H * d);
      sg::moe_group_gemm(g, s);
    }
    {
      Prof pr(D, K_MOE_DOWN_PRE, used * mxfp4_bytes(H * d), 2.0 * n * H * d);
      if (dn.a_hi && !planes) sg::moe_gather_split(dn, s);
      sg::moe_group_gemm(dn, s);
    }
    return true;
  }
  sg::MoeGemvParams g{};
  g.blocks = W8(D, W_GB, l);
  g.scales = W8(D, W_GS, l);
  g.blocks2 = W8(D, W_UB, l);
  g.scales2 = W8(D, W_US, l);
  g.x = D->xn;
  g.expert = D->moe_sel;
  g.logits = fused ? D->moe_logits : nullptr;
  g.E = D->E;
  g.tokens = T;
  g.topk = D->topk;
  g.N = D->H;
  g.K = D->d;
  g.y = D->moe_act;
  {
    Prof pr(D, T == 1 ? K_MOE_GU : K_MOE_GU_PRE, T * k * mxfp4_bytes(2 * H * d), 4.0 * T * k * H * d);
    sg::moe_gemv_swiglu(g, s);
  }
  sg::MoeGemvParams dn{};
  dn.blocks = W8(D, W_DB, l);
  dn.scales = W8(D, W_DS, l);
  dn.x = D->moe_act;
  dn.expert = D->moe_sel;
  dn.weight = D->moe_w;
  dn.logits = fused ? D->moe_logits : nullptr;
  dn.E = D->E;
  dn.tokens = T;
  dn.topk = D->topk;
  dn.N = D->d;
  dn.K = D->H;
  dn.y = D->x;
  {
    Prof pr(D, T == 1 ? K_MOE_DOWN : K_MOE_DOWN_PRE, T * k * mxfp4_bytes(H * d), 2.0 * T * k * H * d);
    sg::moe_gemv_down(dn, s);
  }
  return false;
}

// Layer l's K and V cache bases (fp32 or bf16 elements).
float* kv_layer(const Dev* D, float* base, int l) {
  const size_t cache_layer = (size_t)D->kvh * D->ctx * D->hd;
  return (float*)((char*)base + l * cache_layer * (D->kv_bf16 ? 2 : 4));
}

void layer_decode(Dev* D, int l) {
  hipStream_t s = D->stream;
  float* kc = kv_layer(D, D->kc, l);
  float* vc = kv_layer(D, D->vc, l);
  const double d = D->d;

  sg::GemvParams g{};
  g.w = W16(D, W_Q, l);  // fused QKV block of layer l
  g.x = D->x;
  g.norm_w = W16(D, W_MHA_NORM, l);
  g.eps = D->eps;
  g.N = D->qkv_rows;
  g.K = D->d;
  g.q = D->q;
  g.kraw = D->kraw;
  g.vcache = vc;
  g.pos = D->pos;
  g.q_dim = D->qd;
  g.kv_dim = D->kvd;
  g.head_dim = D->hd;
  g.ctx = D->ctx;
  g.kv_bf16 = D->kv_bf16;
  {
    Prof pr(D, K_QKV_GEMV, (double)D->qkv_rows * d * 2, 2.0 * D->qkv_rows * d);
    sg::gemv(g, sg::GEMV_QKV, s);
  }

  sg::AttnParams a{};
  a.q = D->q;
  a.kcache = kc;
  a.vcache = vc;
  a.out = D->att;
  a.pos = D->pos;
  a.T = 1;
  a.q_heads = D->qh;
  a.kv_heads = D->kvh;
  a.hd = D->hd;
  a.ctx = D->ctx;
  a.kraw = D->kraw;
  a.kcache_w = kc;
  a.kv_bf16 = D->kv_bf16;
  a.qn = D->qk_norm ? W16(D, W_Q_NORM, l) : nullptr;
  a.kn = D->qk_norm ? W16(D, W_K_NORM, l) : nullptr;
  a.eps = D->eps;
  a.rope = D->rope;
  a.pair_bound = D->pb;
  a.pair_offset = D->po;
  a.pair_stride = D->pst;
  {
    const size_t cache_layer = (size_t)D->kvh * D->ctx * D->hd;
    const size_t vt_layer = (size_t)D->kvh * D->hd * D->ctx_pad;
    a.khi = D->kp_hi + l * cache_layer;
    a.klo = D->kp_lo + l * cache_layer;
    a.vthi = D->vt_hi + l * vt_layer;
    a.vtlo = D->vt_lo + l * vt_layer;
    a.ctx_pad = D->ctx_pad;
  }
  a.partial = D->attn_part;
  a.splits = D->attn_splits;
  a.counters = D->attn_cnt;
  {
    const double keys = (double)D->host_pos + 1;
    Prof pr(D, K_ATT_DEC, 2.0 * D->kvh * keys * D->hd * (D->kv_bf16 ? 2 : 4), 4.0 * D->qh * keys * D->hd);
    sg::attention_decode(a, s);
  }

  sg::GemvParams o{};
  o.w = W16(D, W_O, l);
  o.x = D->att;
  o.N = D->d;
  o.K = D->qd;
  o.y = D->x;
  {
    Prof pr(D, K_O_GEMV, d * D->qd * 2, 2.0 * d * D->qd);
    sg::gemv(o, sg::GEMV_RESIDUAL, s);
  }

  if (!D->moe) {
    sg::GemvParams f{};
    f.w = W16(D, W_GATE, l);
    f.w2 = W16(D, W_UP, l);
    f.x = D->x;
    f.norm_w = W16(D, W_FFN_NORM, l);
    f.eps = D->eps;
    f.N = D->H;
    f.K = D->d;
    f.y = D->act;
    {
      Prof pr(D, K_GU_GEMV, 2.0 * D->H * d * 2, 4.0 * D->H * d);
      sg::gemv(f, sg::GEMV_SWIGLU, s);
    }
    sg::GemvParams dn{};
    dn.w = W16(D, W_DOWN, l);
    dn.x = D->act;
    dn.N = D->d;
    dn.K = D->H;
    dn.y = D->x;
    dn.part = D->gemv_part;
    dn.counters = D->gemv_cnt;
    {
      Prof pr(D, K_DOWN_GEMV, d * D->H * 2, 2.0 * d * D->H);
      sg::gemv(dn, sg::GEMV_RESIDUAL, s);
    }
  } else {
    ffn_moe(D, l, 1);
  }
}

// Residual add of a projection (split-K partial sums in D->ws, or already
// added) and the RMSNorm with weight w of the updated rows into the bf16
// planes of the next GEMM (and the fp32 rows for the MoE experts).
void prefill_norm(Dev* D, int T, int splits, const uint16_t* w, bool routed = false) {
  sg::NormParams n{};
  n.x = D->x;
  n.part = splits > 1 ? D->ws : nullptr;
  n.splits = splits > 1 ? splits : 0;
  if (routed) {  // the MoE layer's routed sum, in top-k order
    n.routed = D->moe_out;
    n.routed_w = D->moe_w;
    n.topk = D->topk;
  }
  n.w = w;
  n.eps = D->eps;
  n.rows = T;
  n.d = D->d;
  n.y = D->moe ? D->xn : nullptr;
  n.y_hi = D->xn_hi;
  // (the MoE grouped GEMMs take both planes in either precision)
  n.y_lo = D->precision == sg::GEMM_SPLIT2 || D->moe ? D->xn_lo : nullptr;
  Prof pr(D, K_ELEM, (double)T * D->d * (8 + 4.0 * n.splits), 0);
  sg::residual_norm(n, D->stream);
}

// Projection whose result is added to the residual stream: split-K into
// D->ws when that fills the GPU (summed by the next prefill_norm), else a
// direct residual epilogue. Returns the split count.
int residual_gemm(Dev* D, const uint16_t* a_hi, const uint16_t* a_lo, int lda,
                  const uint16_t* w, int T, int N, int K, int cls) {
  sg::GemmParams g{};
  g.a_hi = a_hi;
  g.a_lo = a_lo;
  g.lda = lda;
  g.w = w;
  g.M = T;
  g.N = N;
  g.K = K;
  g.ldc = N;
  int splits = sg::gemm_splits(T, N, K);
  if (splits > D->ws_splits) splits = D->ws_splits;
  if (splits > 1 && (size_t)splits * T > (size_t)D->ws_splits * D->ws_rows)
    splits = (int)std::max<size_t>(1, (size_t)D->ws_splits * D->ws_rows / T);
  Prof pr(D, cls, (double)N * K * 2, 2.0 * T * N * K);
  if (splits > 1) {
    g.c = D->ws;
    sg::gemm(g, sg::GEMM_PARTIAL, D->precision, splits, D->stream);
  } else {
    g.c = D->x;
    sg::gemm(g, sg::GEMM_RESIDUAL, D->precision, 1, D->stream);
  }
  return splits;
}

// Queries per prefill attention launch (measured on the 8192-token chunk):
// 512 for the fp32 kernel (one block per CU: a launch over a long chunk
// balances its causal ranges less well); the whole chunk for the split-bf16
// kernel, whose blocks go out longest causal range first across all heads
// (2048, 4096, 8192 queries per launch: 1.82, 1.66, 1.59 ms per layer; 512:
// 3.5 ms, half the CUs empty). STRASGPT_ATTN_ROWS overrides (>= 64).
int attn_rows() {
  const char* e = getenv("STRASGPT_ATTN_ROWS");
  if (e && *e) {
    const int v = atoi(e);
    if (v < 64) ST_DIE("STRASGPT_ATTN_ROWS must be at least 64");
    return v;
  }
  const char* k = getenv("STRASGPT_PREFILL_ATTN");
  return k && !strcmp(k, "fp32") ? 512 : 1 << 30;
}

// One layer over T > 1 rows. On entry D->xn_hi/lo hold the layer's input
// RMSNorm; on exit x holds the layer output and, if next_norm is given, the
// planes hold its RMSNorm with that weight.
void layer_prefill(Dev* D, int l, int T, const uint16_t* next_norm) {
  hipStream_t s = D->stream;
  const size_t cache_layer = (size_t)D->kvh * D->ctx * D->hd;
  float* kc = kv_layer(D, D->kc, l);
  float* vc = kv_layer(D, D->vc, l);
  const double d = D->d, M = T;
  const bool split = D->precision == sg::GEMM_SPLIT2;

  sg::GemmParams g{};
  g.a_hi = D->xn_hi;
  g.a_lo = split ? D->xn_lo : nullptr;
  g.lda = D->d;
  g.w = W16(D, W_Q, l);
  g.M = T;
  g.N = D->qkv_rows;
  g.K = D->d;
  g.q = D->q;
  g.kcache = kc;
  g.vcache = vc;
  g.pos = D->pos;
  g.q_dim = D->qd;
  g.kv_dim = D->kvd;
  g.head_dim = D->hd;
  g.ctx = D->ctx;
  g.kv_bf16 = D->kv_bf16;
  g.kstage = D->kv_bf16 ? D->kstage : nullptr;
  {
    Prof pr(D, K_QKV_GEMM, (double)D->qkv_rows * d * 2, 2.0 * M * D->qkv_rows * d);
    const size_t ws_floats = (size_t)D->ws_splits * D->ws_rows * D->d;
    const int sp = sg::gemm_small_splits(T, D->qkv_rows, D->d, sg::GEMM_QKV, ws_floats);
    if (sp > 1) sg::gemm_small(g, sg::GEMM_QKV, D->precision, sp, D->ws, s);
    else sg::gemm(g, sg::GEMM_QKV, D->precision, 1, s);
  }
  {
    Prof pr(D, K_ELEM, 2.0 * M * (D->qd + D->kvd) * 4, 0);
    sg::qk_norm_rope(D->q, D->qh, kc, D->kvh, T, D->pos, D->ctx, D->hd,
                     D->qk_norm ? W16(D, W_Q_NORM, l) : nullptr,
                     D->qk_norm ? W16(D, W_K_NORM, l) : nullptr, D->eps, D->rope, D->pb,
                     D->po, D->pst, D->kv_bf16 ? D->kstage : nullptr, nullptr, s);
  }
  // this chunk's cache rows into the bf16 planes (from a multiple of 32;
  // decode steps write their rows into the planes themselves)
  const size_t P0 = D->host_pos;
  const size_t vt_layer = (size_t)D->kvh * D->hd * D->ctx_pad;
  {
    const int r0 = (int)(P0 / 32 * 32), r1 = (int)(P0 + T);
    Prof pr(D, K_ELEM, 2.0 * (r1 - r0) * D->kvd * 4 * 2, 0);
    sg::attention_split_rows(kc, vc, D->kp_hi + l * cache_layer, D->kp_lo + l * cache_layer,
                             D->vt_hi + l * vt_layer, D->vt_lo + l * vt_layer, D->kvh, D->ctx,
                             D->ctx_pad, D->hd, r0, r1, D->kv_bf16, s);
  }
  sg::AttnParams a{};
  a.q = D->q;
  a.kcache = kc;
  a.vcache = vc;
  a.kv_bf16 = D->kv_bf16;
  a.khi = D->kp_hi + l * cache_layer;
  a.klo = D->kp_lo + l * cache_layer;
  a.vthi = D->vt_hi + l * vt_layer;
  a.vtlo = D->vt_lo + l * vt_layer;
  a.ctx_pad = D->ctx_pad;
  a.out_hi = D->att_hi;
  a.out_lo = split ? D->att_lo : nullptr;
  a.pos = D->pos;
  a.T = T;
  a.q_heads = D->qh;
  a.kv_heads = D->kvh;
  a.hd = D->hd;
  a.ctx = D->ctx;
  {
    // causal (query, key) pairs: sum over t of (P + t + 1)
    const double pairs = M * (double)D->host_pos + M * (M + 1) / 2;
    Prof pr(D, K_ATT_PRE, 2.0 * D->kvh * ((double)D->host_pos + M) * D->hd * (D->kv_bf16 ? 2 : 4),
            4.0 * D->qh * D->hd * pairs);
    // launches of at most attn_rows() queries
    const int rows = attn_rows();
    for (int q0 = 0; q0 < T; q0 += rows) {
      sg::AttnParams b = a;
      b.q0 = q0;
      b.T = std::min(rows, T - q0);
      b.q = D->q + (size_t)q0 * D->qd;
      b.out_hi = D->att_hi + (size_t)q0 * D->qd;
      b.out_lo = split ? D->att_lo + (size_t)q0 * D->qd : nullptr;
      sg::attention_prefill(b, s);
    }
  }
  const int so = residual_gemm(D, D->att_hi, split ? D->att_lo : nullptr, D->qd, W16(D, W_O, l),
                               T, D->d, D->qd, K_O_GEMM);
  prefill_norm(D, T, so, W16(D, W_FFN_NORM, l));
  if (!D->moe) {
    sg::GemmParams f{};
    f.a_hi = D->xn_hi;
    f.a_lo = split ? D->xn_lo : nullptr;
    f.lda = D->d;
    f.w = W16(D, W_GATE, l);
    f.w2 = W16(D, W_UP, l);
    f.M = T;
    f.N = D->H;
    f.K = D->d;
    f.ldc = D->H;
    f.c_hi = D->act_hi;
    f.c_lo = split ? D->act_lo : nullptr;
    {
      Prof pr(D, K_GU_GEMM, 2.0 * D->H * d * 2, 4.0 * M * D->H * d);
      // (the split form measured slower here: two partial GEMMs and the
      // epilogue took 32 us against 23 for the fused GEMM at 8 rows)
      sg::gemm(f, sg::GEMM_SWIGLU, D->precision, 1, s);
    }
    const int sd = residual_gemm(D, D->act_hi, split ? D->act_lo : nullptr, D->H,
                                 W16(D, W_DOWN, l), T, D->d, D->H, K_DOWN_GEMM);
    prefill_norm(D, T, sd, next_norm);
  } else {
    const bool routed = ffn_moe(D, l, T);
    prefill_norm(D, T, 0, next_norm, routed);
  }
}

// Prompts of at most sg::kRowsMax tokens on dense models: the projections
// as multi-row GEMVs (each weight row streamed once into fp32 FMAs for all
// rows, the RMSNorms fused in; the residual stream x stays fp32 and is
// updated in place), attention as in layer_prefill with fp32 output rows.
// STRASGPT_PREFILL_ROWS=0 keeps such prompts on the GEMMs.
bool prefill_rows(Dev* D, int T) {
  const char* e = getenv("STRASGPT_PREFILL_ROWS");
  const bool off = e && !strcmp(e, "0");
  return !off && !D->moe && T >= 2 && T <= sg::kRowsMax && D->precision == sg::GEMM_SPLIT2 &&
         sg::gemv_rows_fit(T, D->d, true) && sg::gemv_rows_fit(T, D->qd, false) &&
         sg::gemv_rows_fit(T, D->H, false);
}

void layer_prefill_rows(Dev* D, int l, int T) {
  hipStream_t s = D->stream;
  const size_t cache_layer = (size_t)D->kvh * D->ctx * D->hd;
  float* kc = kv_layer(D, D->kc, l);
  float* vc = kv_layer(D, D->vc, l);
  const double d = D->d, M = T;
  auto need = [](bool ok) {
    if (!ok) ST_DIE("multi-row GEMV refused a shape it was planned for");
  };

  sg::GemvParams g{};
  g.w = W16(D, W_Q, l);
  g.x = D->x;
  g.norm_w = W16(D, W_MHA_NORM, l);
  g.eps = D->eps;
  g.N = D->qkv_rows;
  g.K = D->d;
  g.M = T;
  g.q = D->q;
  g.kcache = kc;
  g.kstage = D->kv_bf16 ? D->kstage : nullptr;
  g.vcache = vc;
  g.pos = D->pos;
  g.q_dim = D->qd;
  g.kv_dim = D->kvd;
  g.head_dim = D->hd;
  g.ctx = D->ctx;
  g.kv_bf16 = D->kv_bf16;
  {
    Prof pr(D, K_QKV_GEMM, (double)D->qkv_rows * d * 2, 2.0 * M * D->qkv_rows * d);
    need(sg::gemv_rows(g, sg::GEMV_QKV, s));
  }
  // the prompt's cache rows go into the bf16 planes with the keys' norm and
  // rotation (rows before P0 are there already: earlier chunks and decode
  // steps write theirs), else, where that kernel cannot, by split_rows
  const size_t P0 = D->host_pos;
  const size_t vt_layer = (size_t)D->kvh * D->hd * D->ctx_pad;
  bool planes_done;
  {
    Prof pr(D, K_ELEM, 2.0 * M * (D->qd + D->kvd) * 4, 0);
    const sg::PlaneRows pl{D->kp_hi + l * cache_layer, D->kp_lo + l * cache_layer, D->vt_hi + l * vt_layer,
                           D->vt_lo + l * vt_layer, vc, D->ctx_pad, D->kv_bf16};
    planes_done = sg::qk_norm_rope(D->q, D->qh, kc, D->kvh, T, D->pos, D->ctx, D->hd,
                                   D->qk_norm ? W16(D, W_Q_NORM, l) : nullptr,
                                   D->qk_norm ? W16(D, W_K_NORM, l) : nullptr, D->eps, D->rope, D->pb,
                                   D->po, D->pst, D->kv_bf16 ? D->kstage : nullptr, &pl, s);
  }
  if (!planes_done) {
    const int r0 = (int)(P0 / 32 * 32), r1 = (int)(P0 + T);
    Prof pr(D, K_ELEM, 2.0 * (r1 - r0) * D->kvd * 4 * 2, 0);
    sg::attention_split_rows(kc, vc, D->kp_hi + l * cache_layer, D->kp_lo + l * cache_layer,
                             D->vt_hi + l * vt_layer, D->vt_lo + l * vt_layer, D->kvh, D->ctx,
                             D->ctx_pad, D->hd, r0, r1, D->kv_bf16, s);
  }
  sg::AttnParams a{};
  a.q = D->q;
  a.kcache = kc;
  a.vcache = vc;
  a.kv_bf16 = D->kv_bf16;
  a.khi = D->kp_hi + l * cache_layer;
  a.klo = D->kp_lo + l * cache_layer;
  a.vthi = D->vt_hi + l * vt_layer;
  a.vtlo = D->vt_lo + l * vt_layer;
  a.ctx_pad = D->ctx_pad;
  a.out = D->att;  // fp32 rows [T][qd]
  a.pos = D->pos;
  a.T = T;
  a.q_heads = D->qh;
  a.kv_heads = D->kvh;
  a.hd = D->hd;
  a.ctx = D->ctx;
  {
    const double pairs = M * (double)D->host_pos + M * (M + 1) / 2;
    Prof pr(D, K_ATT_PRE, 2.0 * D->kvh * ((double)D->host_pos + M) * D->hd * (D->kv_bf16 ? 2 : 4),
            4.0 * D->qh * D->hd * pairs);
    sg::attention_prefill(a, s);
  }
  sg::GemvParams o{};
  o.w = W16(D, W_O, l);
  o.x = D->att;
  o.N = D->d;
  o.K = D->qd;
  o.M = T;
  o.y = D->x;
  o.part = D->ws;
  o.counters = D->gemv_cnt;
  {
    Prof pr(D, K_O_GEMM, (double)D->qd * d * 2, 2.0 * M * D->qd * d);
    need(sg::gemv_rows(o, sg::GEMV_RESIDUAL, s));
  }
  sg::GemvParams f{};
  f.w = W16(D, W_GATE, l);
  f.w2 = W16(D, W_UP, l);
  f.x = D->x;
  f.norm_w = W16(D, W_FFN_NORM, l);
  f.eps = D->eps;
  f.N = D->H;
  f.K = D->d;
  f.M = T;
  f.y = D->act;  // [T][H]
  {
    Prof pr(D, K_GU_GEMM, 2.0 * D->H * d * 2, 4.0 * M * D->H * d);
    need(sg::gemv_rows(f, sg::GEMV_SWIGLU, s));
  }
  sg::GemvParams dn{};
  dn.w = W16(D, W_DOWN, l);
  dn.x = D->act;
  dn.N = D->d;
  dn.K = D->H;
  dn.M = T;
  dn.y = D->x;
  dn.part = D->ws;
  dn.counters = D->gemv_cnt;
  {
    Prof pr(D, K_DOWN_GEMM, (double)D->H * d * 2, 2.0 * M * D->H * d);
    need(sg::gemv_rows(dn, sg::GEMV_RESIDUAL, s));
  }
}

// Logits of chunk rows [T - lc, T): final RMSNorm fused into the GEMV.
void classifier(Dev* D, int T, int lc) {
  for (int r = 0; r < lc; r++) {
    sg::GemvParams g{};
    g.w = D->tied ? W16(D, W_EMB) : W16(D, W_OUT);
    g.x = D->x + (size_t)(T - lc + r) * D->d;
    g.norm_w = W16(D, W_OUT_NORM);
    g.eps = D->eps;
    g.N = D->V;
    g.K = D->d;
    g.y = D->logits + (size_t)r * D->V;
    Prof pr(D, K_LOGITS, (double)D->V * D->d * 2, 2.0 * D->V * D->d);
    sg::gemv(g, sg::GEMV_STORE, D->stream);
  }
}

// One chunk of T <= D->chunk tokens whose ids are in device memory at `tok`,
// at the device position *D->pos (mirrored on the host in D->host_pos).
void forward_chunk(Dev* D, const int* tok, int T, int lc) {
  {
    Prof pr(D, K_ELEM, (double)T * D->d * 6, 0);
    sg::embed(tok, T, W16(D, W_EMB), D->d, D->x, D->stream);
  }
  const bool capture = D->cap_out != nullptr;
  const bool rows = T > 1 && prefill_rows(D, T);
  if (T > 1 && !rows) prefill_norm(D, T, 0, W16(D, W_MHA_NORM, 0));
  for (int l = 0; l < D->L; l++) {
    if (T == 1) layer_decode(D, l);
    else if (rows) layer_prefill_rows(D, l, T);
    else layer_prefill(D, l, T, l + 1 < D->L ? W16(D, W_MHA_NORM, l + 1) : nullptr);
    if (capture)
      HIP_CHECK(hipMemcpyAsync(D->cap_dev + (size_t)l * T * D->d, D->x,
                               (size_t)T * D->d * sizeof(float), hipMemcpyDeviceToDevice,
                               D->stream));
  }
  if (capture) sg::rmsnorm_rows(D->x, W16(D, W_OUT_NORM), D->cap_final_dev, T, D->d, D->eps, D->stream);
  if (lc > 0) classifier(D, T, lc);
}

void ensure_logits(Dev* D, int rows) {
  if (rows <= D->logits_rows) return;
  HIP_CHECK(hipStreamSynchronize(D->stream));
  if (D->graph || D->graph_body) {  // the captured decode step points at the old buffer
    drop_graphs(D);
  }
  if (D->logits) HIP_CHECK(hipFree(D->logits));
  D->logits = dalloc<float>((size_t)rows * D->V);
  D->logits_rows = rows;
}

void set_pos(Dev* D, size_t pos) {
  *D->h_pos = (int)pos;
  D->host_pos = pos;
  HIP_CHECK(hipMemcpyAsync(D->pos, D->h_pos, sizeof(int), hipMemcpyHostToDevice, D->stream));
}

void upload_tokens(Dev* D, const int* token, int T) {
  for (int i = 0; i < T; i++) {
    if (token[i] < 0 || token[i] >= D->V) ST_DIE("token id out of range");
    D->h_tok[i] = token[i];
  }
  HIP_CHECK(hipMemcpyAsync(D->tok, D->h_tok, (size_t)T * sizeof(int), hipMemcpyHostToDevice,
                           D->stream));
}

void argmax_to(Dev* D, const float* row, bool log_seq, bool bump_pos) {
  sg::ArgmaxParams p{};
  p.x = row;
  p.n = D->V;
  p.part_v = D->am_v;
  p.part_i = D->am_i;
  p.out = D->next;
  p.seq = log_seq ? D->seq : nullptr;
  p.seq_len = log_seq ? D->seq_len : nullptr;
  p.pos_inc = bump_pos ? D->pos : nullptr;
  Prof pr(D, K_ARGMAX, (double)D->V * 4, 0);
  sg::argmax(p, D->stream);
}

// The reference chunk loop over `token` (source/transformer.c:1643-1726):
// logits of the caller's window [T - lc, T) are copied to host_logits (if
// given); the last chunk's rows stay on the device.
void predict_device(transformer_t* t, size_t T, const int* token, size_t lc,
                    float* host_logits) {
  Dev* D = t->device;
  if (T + t->state->cached_count > (size_t)D->ctx) ST_DIE("context length exhausted");
  if (lc > T) lc = T;
  const size_t start = T - lc;
  // The device runs prompts in chunks of D->chunk rows (the results do not
  // depend on the chunk length: every row attends to the cache before its
  // chunk and causally within it); hidden-state capture keeps the API's
  // 512-token chunk.
  const size_t chunk_max = D->cap_out ? (size_t)TRANSFORMER_CHUNK_MAX_LEN : D->chunk;
  if (D->cap_out && T > chunk_max) ST_DIE("hidden-state capture covers one chunk of at most 512 tokens");
  for (size_t c0 = 0; c0 < T; c0 += chunk_max) {
    const size_t n = T - c0 < chunk_max ? T - c0 : chunk_max;
    const size_t lo = c0 > start ? c0 : start, hi = c0 + n;
    const size_t clc = lo < hi ? hi - lo : 0;
    ensure_logits(D, (int)(clc > 0 ? clc : 1));
    upload_tokens(D, token + c0, (int)n);
    set_pos(D, t->state->cached_count);
    forward_chunk(D, D->tok, (int)n, (int)clc);
    if (clc > 0 && host_logits) {
      HIP_CHECK(hipMemcpyAsync(host_logits + (lo - start) * D->V, D->logits,
                               clc * D->V * sizeof(float), hipMemcpyDeviceToHost, D->stream));
    }
    HIP_CHECK(hipStreamSynchronize(D->stream));
    harvest(D);
    t->state->cached_count += n;
  }
  if (D->cap_out) {
    HIP_CHECK(hipMemcpy(D->cap_out, D->cap_dev, (size_t)D->L * T * D->d * sizeof(float),
                        hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(D->cap_final, D->cap_final_dev, T * D->d * sizeof(float),
                        hipMemcpyDeviceToHost));
    D->cap_out = nullptr;
    D->cap_final = nullptr;
  }
}

void build_decode_graph(Dev* D, bool with_argmax = true) {
  if (with_argmax ? D->graph != nullptr : D->graph_body != nullptr) return;
  hipGraph_t g;
  float* cap = D->cap_out;  // hidden-state capture is never part of the graph
  D->cap_out = nullptr;
  HIP_CHECK(hipStreamBeginCapture(D->stream, hipStreamCaptureModeRelaxed));
  forward_chunk(D, D->next, 1, 1);
  if (with_argmax) argmax_to(D, D->logits, true, true);
  HIP_CHECK(hipStreamEndCapture(D->stream, &g));
  D->cap_out = cap;
  HIP_CHECK(hipGraphInstantiate(with_argmax ? &D->graph : &D->graph_body, g, nullptr, nullptr, 0));
  HIP_CHECK(hipGraphDestroy(g));
}

}  // namespace

// ================================================================= API ==

extern "C" transformer_t* sg_from_safetensors(struct safetensors* st) {
  if (!st) ST_DIE("NULL safetensors");
  transformer_t* t = (transformer_t*)calloc(1, sizeof(transformer_t));
  transformer_configuration_t* c =
      (transformer_configuration_t*)calloc(1, sizeof(transformer_configuration_t));
  transformer_weights_t* w = (transformer_weights_t*)calloc(1, sizeof(transformer_weights_t));
  transformer_state_t* ss = (transformer_state_t*)calloc(1, sizeof(transformer_state_t));
  Dev* D = new Dev();
  if (!t || !c || !w || !ss) ST_DIE("failed to malloc for transformer_t");
  t->config = c;
  t->weights = w;
  t->state = ss;
  t->device = D;

  // Configuration (reference configuration_from_safetensors,
  // source/transformer.c:17-58).
  c->embedding_dim = st->embedding_dim;
  c->head_dim = st->head_dim;
  c->hidden_dim = st->hidden_dim;
  c->layer_count = st->layer_count;
  c->q_head_count = st->q_head_count;
  c->kv_head_count = st->kv_head_count;
  c->vocabulary_len = st->vocabulary_len;
  c->context_len = st->context_len;
  c->epsilon = st->epsilon;
  c->rope_theta = st->rope_theta;
  if (st->rope_interleaved) {
    c->rope_pair_bound = st->head_dim;
    c->rope_pair_offset = 1;
    c->rope_pair_stride = 2;
  } else {
    c->rope_pair_bound = st->head_dim / 2;
    c->rope_pair_offset = st->head_dim / 2;
    c->rope_pair_stride = 1;
  }
  c->mrope_section_count = st->mrope_section_count;
  if (c->mrope_section_count) {
    c->mrope_section = (size_t*)calloc(c->mrope_section_count, sizeof(size_t));
    for (size_t i = 0; i < c->mrope_section_count; i++) c->mrope_section[i] = st->mrope_section[i];
  }
  c->aliased_out_weight = safetensors_aliased_out_weight(st);
  c->qk_norm = has_tensor(st, W_Q_NORM);
  const bool moe = has_tensor(st, W_ROUTER);
  c->expert_count = moe ? st->expert_count : 0;
  c->expert_used_count = moe ? st->expert_used_count : 0;

  D->d = (int)c->embedding_dim;
  D->hd = (int)c->head_dim;
  D->H = (int)c->hidden_dim;
  D->L = (int)c->layer_count;
  D->qh = (int)c->q_head_count;
  D->kvh = (int)c->kv_head_count;
  D->V = (int)c->vocabulary_len;
  D->ctx = (int)c->context_len;
  D->qd = D->qh * D->hd;
  D->kvd = D->kvh * D->hd;
  D->qkv_rows = D->qd + 2 * D->kvd;
  D->eps = c->epsilon;
  D->qk_norm = c->qk_norm;
  D->moe = moe;
  D->tied = c->aliased_out_weight;
  D->E = (int)c->expert_count;
  D->topk = (int)c->expert_used_count;
  D->pb = (int)c->rope_pair_bound;
  D->po = (int)c->rope_pair_offset;
  D->pst = (int)c->rope_pair_stride;

  if (!D->d || !D->hd || !D->H || !D->L || !D->qh || !D->kvh || !D->V || !D->ctx)
    ST_DIE("incomplete model configuration");
  if (D->qh % D->kvh) ST_DIE("q_head_count must be a multiple of kv_head_count");
  if (D->d % 32 || D->H % 32 || D->qd % 32) ST_DIE("model dimensions must be multiples of 32");
  if (D->hd != 16 && D->hd != 32 && D->hd != 64 && D->hd != 128)
    ST_DIE("head_dim must be 16, 32, 64 or 128");
  if (moe && (D->E <= 0 || D->topk <= 0 || D->topk > D->E || D->E > 1024))
    ST_DIE("MoE model needs num_local_experts and num_experts_per_tok");

  HIP_CHECK(hipStreamCreateWithFlags(&D->stream, hipStreamNonBlocking));
  {
    const char* g = getenv("STRASGPT_DECODE_GRAPH");
    D->use_graph = !(g && g[0] == '0');
  }

  // Per-layer byte sizes of each weight class.
  const size_t d = D->d, hd = D->hd, H = D->H, E = D->E, V = D->V;
  size_t* pl = D->per_layer;
  pl[W_EMB] = V * d * 2;
  pl[W_MHA_NORM] = d * 2;
  pl[W_Q] = (size_t)D->qkv_rows * d * 2;  // fused Q|K|V block
  pl[W_Q_NORM] = c->qk_norm ? hd * 2 : 0;
  pl[W_K_NORM] = c->qk_norm ? hd * 2 : 0;
  pl[W_O] = d * D->qd * 2;
  pl[W_FFN_NORM] = d * 2;
  pl[W_GATE] = moe ? 0 : H * d * 2;
  pl[W_UP] = moe ? 0 : H * d * 2;
  pl[W_DOWN] = moe ? 0 : d * H * 2;
  pl[W_OUT_NORM] = d * 2;
  pl[W_OUT] = D->tied ? 0 : V * d * 2;
  pl[W_ROUTER] = E * d * 2;
  pl[W_GB] = pl[W_UB] = E * H * d / 2;
  pl[W_GS] = pl[W_US] = E * H * d / 32;
  pl[W_DB] = E * d * H / 2;
  pl[W_DS] = E * d * H / 32;
  for (int k = 0; k < W_COUNT; k++) {
    if (!pl[k]) continue;
    const size_t layers = is_global(k) ? 1 : (size_t)D->L;
    D->w[k] = dalloc<uint8_t>(pl[k] * layers);
  }
  if (D->tied) D->w[W_OUT] = D->w[W_EMB];

  // Expected tensor size for each class (K and V share the fused block).
  auto expect = [&](int cls) -> size_t {
    if (cls == W_Q) return (size_t)D->qd * d * 2;
    if (cls == W_K || cls == W_V) return (size_t)D->kvd * d * 2;
    return pl[cls];
  };
  auto dest = [&](int cls, long l) -> char* {
    if (cls == W_Q) return (char*)D->w[W_Q] + l * pl[W_Q];
    if (cls == W_K) return (char*)D->w[W_Q] + l * pl[W_Q] + (size_t)D->qd * d * 2;
    if (cls == W_V) return (char*)D->w[W_Q] + l * pl[W_Q] + (size_t)(D->qd + D->kvd) * d * 2;
    return (char*)D->w[cls] + l * pl[cls];
  };

  std::vector<std::vector<char>> seen(W_COUNT + 2);
  for (int k = 0; k < W_COUNT + 2; k++) seen[k].assign(k < W_COUNT && is_global(k) ? 1 : D->L, 0);
  std::vector<int> fds(st->file_count, -1);
  {
    Stager stage(D->stream);
    for (size_t i = 0; i < st->tensor_count; i++) {
      const safetensors_tensor_t* tn = &st->tensor[i];
      WClass cls;
      long layer;
      if (!classify(tn->name, &cls, &layer) ||
          (cls != W_K && cls != W_V && !pl[cls] && !(cls == W_OUT && !D->tied))) {
        fprintf(stderr, "[StrasGPT] Warning: unknown tensor %s\n", tn->name);
        continue;
      }
      if (layer < 0 || layer >= (is_global(cls) ? 1 : D->L)) ST_DIE("tensor layer index out of range");
      const bool u8 = cls >= W_GB;
      if (tn->type != (u8 ? SAFETENSORS_TYPE_U8 : SAFETENSORS_TYPE_BF16)) {
        char m[SAFETENSORS_MAX_STRING];
        snprintf(m, sizeof(m), "unexpected dtype for %s", tn->name);
        ST_DIE(m);
      }
      if (tn->size != expect(cls)) {
        char m[SAFETENSORS_MAX_STRING];
        snprintf(m, sizeof(m), "unexpected size for %s: have %zu expected %zu", tn->name,
                 tn->size, expect(cls));
        ST_DIE(m);
      }
      if (tn->file >= st->file_count) ST_DIE("tensor file index out of range");
      if (fds[tn->file] < 0) {
        fds[tn->file] = open(st->file[tn->file], O_RDONLY);
        if (fds[tn->file] < 0) ST_DIE("failed to open file");
      }
      stage.copy(fds[tn->file], tn->offset, tn->size, dest(cls, layer));
      const int slot = (cls == W_K) ? W_COUNT : (cls == W_V) ? W_COUNT + 1 : cls;
      seen[slot][layer] = 1;
    }
  }
  for (int fd : fds)
    if (fd >= 0) close(fd);
  for (int k = 0; k < W_COUNT + 2; k++) {
    const bool needed = k >= W_COUNT || (pl[k] && !(k == W_OUT && D->tied));
    if (!needed) continue;
    for (size_t l = 0; l < seen[k].size(); l++) {
      if (!seen[k][l]) {
        char m[256];
        snprintf(m, sizeof(m), "missing tensor: %s of layer %zu",
                 k == W_COUNT ? "mha_k" : k == W_COUNT + 1 ? "mha_v" : kClassName[k], l);
        ST_DIE(m);
      }
    }
  }

  // Public weight pointers.
  w->embedding_weight = W16(D, W_EMB);
  w->mha_norm_weight = W16(D, W_MHA_NORM);
  w->mha_qkv_weight = W16(D, W_Q);
  w->mha_q_norm_weight = c->qk_norm ? W16(D, W_Q_NORM) : nullptr;
  w->mha_k_norm_weight = c->qk_norm ? W16(D, W_K_NORM) : nullptr;
  w->mha_out_weight = W16(D, W_O);
  w->ffn_norm_weight = W16(D, W_FFN_NORM);
  w->ffn_fc_weight = moe ? nullptr : W16(D, W_GATE);
  w->ffn_up_weight = moe ? nullptr : W16(D, W_UP);
  w->ffn_out_weight = moe ? nullptr : W16(D, W_DOWN);
  w->out_norm_weight = W16(D, W_OUT_NORM);
  w->out_weight = W16(D, W_OUT);
  if (moe) {
    w->moe_router_weight = W16(D, W_ROUTER);
    w->moe_gate_blocks = W8(D, W_GB);
    w->moe_gate_scales = W8(D, W_GS);
    w->moe_up_blocks = W8(D, W_UB);
    w->moe_up_scales = W8(D, W_US);
    w->moe_down_blocks = W8(D, W_DB);
    w->moe_down_scales = W8(D, W_DS);
  }

  // Host-side summaries for transformer_print (first/last values).
  for (int k = 0; k < W_COUNT; k++) {
    Summary& sm = D->summary[k];
    if (!D->w[k] || (k == W_OUT && D->tied)) continue;
    sm.present = true;
    sm.bytes = pl[k] * (is_global(k) ? 1 : D->L);
    if (k >= W_GB) continue;
    uint16_t head[3], tail[3];
    HIP_CHECK(hipMemcpy(head, D->w[k], sizeof(head), hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(tail, (char*)D->w[k] + sm.bytes - sizeof(tail), sizeof(tail),
                        hipMemcpyDeviceToHost));
    for (int i = 0; i < 3; i++) {
      uint32_t a = (uint32_t)head[i] << 16, b = (uint32_t)tail[i] << 16;
      memcpy(&sm.first[i], &a, 4);
      memcpy(&sm.last[i], &b, 4);
    }
  }

  // State. Prefill chunk: STRASGPT_PREFILL_CHUNK rows (default 8192; at
  // least the API's 512, at most the context): larger chunks give the
  // prefill GEMMs larger M (wider tiles) and fewer launches.
  {
    size_t ch = 8192;
    if (const char* v = getenv("STRASGPT_PREFILL_CHUNK")) ch = (size_t)strtoull(v, nullptr, 10);
    if (ch < TRANSFORMER_CHUNK_MAX_LEN) ch = TRANSFORMER_CHUNK_MAX_LEN;
    if (ch > (size_t)D->ctx) ch = std::max<size_t>(D->ctx, TRANSFORMER_CHUNK_MAX_LEN);
    D->chunk = ch;
  }
  const size_t T = D->chunk;
  const size_t wide = H > d ? H : d;
  D->x = dalloc<float>(T * d);
  D->xn = dalloc<float>(T * wide);
  D->q = dalloc<float>(T * D->qd);
  D->att = dalloc<float>(T * D->qd);
  D->act = dalloc<float>(T * wide);
  D->kraw = dalloc<float>(D->kvd);
  D->xn_hi = dalloc<uint16_t>(T * d);
  D->xn_lo = dalloc<uint16_t>(T * d);
  D->att_hi = dalloc<uint16_t>(T * D->qd);
  D->att_lo = dalloc<uint16_t>(T * D->qd);
  D->act_hi = dalloc<uint16_t>(T * H);
  D->act_lo = dalloc<uint16_t>(T * H);
  // split-K workspace: up to 8 splits of a 512-row chunk, 4 of a full chunk
  // (long reductions such as a 32768-wide down projection split 3 ways)
  D->ws_splits = 8;
  D->ws_rows = std::max<size_t>(TRANSFORMER_CHUNK_MAX_LEN, T / 2);
  D->ws = dalloc<float>((size_t)D->ws_splits * D->ws_rows * d);
  const size_t cache = (size_t)D->L * D->kvh * D->ctx * hd;
  {
    const char* f = getenv("STRASGPT_KV_CACHE");
    if (f && *f && strcmp(f, "fp32") && strcmp(f, "bf16")) ST_DIE("STRASGPT_KV_CACHE must be fp32 or bf16");
    D->kv_bf16 = f && !strcmp(f, "bf16");
  }
  alloc_kv(D, cache);
  D->ctx_pad = (D->ctx + 31) / 32 * 32;
  {
    const size_t kn = cache, vn = (size_t)D->L * D->kvh * D->hd * D->ctx_pad;
    D->kp_hi = dalloc<uint16_t>(kn);
    D->kp_lo = dalloc<uint16_t>(kn);
    D->vt_hi = dalloc<uint16_t>(vn);
    D->vt_lo = dalloc<uint16_t>(vn);
    HIP_CHECK(hipMemsetAsync(D->kp_hi, 0, kn * 2, D->stream));
    HIP_CHECK(hipMemsetAsync(D->kp_lo, 0, kn * 2, D->stream));
    HIP_CHECK(hipMemsetAsync(D->vt_hi, 0, vn * 2, D->stream));
    HIP_CHECK(hipMemsetAsync(D->vt_lo, 0, vn * 2, D->stream));
  }
  std::vector<float> rope;
  build_rope_table(c, rope);
  D->rope = dalloc<float>(rope.size());
  HIP_CHECK(hipMemcpy(D->rope, rope.data(), rope.size() * sizeof(float), hipMemcpyHostToDevice));
  D->tok = dalloc<int>(T);
  D->pos = dalloc<int>(1);
  D->next = dalloc<int>(1);
  D->seq_cap = D->ctx + 1;
  D->seq = dalloc<int>(D->seq_cap);
  D->seq_len = dalloc<int>(1);
  D->attn_splits = sg::attention_decode_chunks(D->kvh);
  D->attn_part = dalloc<float>((size_t)D->qh * D->attn_splits * (hd + 2));
  D->attn_cnt = dalloc<unsigned>(D->kvh);
  HIP_CHECK(hipMemset(D->attn_cnt, 0, D->kvh * sizeof(unsigned)));
  D->gemv_part = dalloc<float>((size_t)8 * D->d);
  D->gemv_cnt = dalloc<unsigned>(sg::kGemvCounters);
  HIP_CHECK(hipMemset(D->gemv_cnt, 0, sg::kGemvCounters * sizeof(unsigned)));
  sg::attention_init();
  D->am_v = dalloc<float>(sg::argmax_blocks());
  D->am_i = dalloc<int>(sg::argmax_blocks());
  if (moe) {
    D->moe_sel = dalloc<int>(T * D->topk);
    D->moe_w = dalloc<float>(T * D->topk);
    D->moe_act = dalloc<float>(T * D->topk * H);
    D->moe_logits = dalloc<float>(D->E);
    // all-zero router logits select experts 0 .. topk-1 (ties go to the
    // lowest id) until a decode step writes them
    HIP_CHECK(hipMemsetAsync(D->moe_logits, 0, D->E * sizeof(float), D->stream));
    D->moe_offs = dalloc<int>(D->E + 1);
    D->moe_order = dalloc<int>(T * D->topk);
    D->moe_out = dalloc<float>(T * D->topk * d);
    D->moe_ahi = dalloc<uint16_t>((size_t)T * D->topk * std::max(d, H));
    D->moe_alo = dalloc<uint16_t>((size_t)T * D->topk * std::max(d, H));
  }
  HIP_CHECK(hipHostMalloc((void**)&D->h_tok, T * sizeof(int), hipHostMallocDefault));
  HIP_CHECK(hipHostMalloc((void**)&D->h_pos, sizeof(int), hipHostMallocDefault));
  HIP_CHECK(hipHostMalloc((void**)&D->h_next, sizeof(int), hipHostMallocDefault));
  ensure_logits(D, 1);
  HIP_CHECK(hipStreamSynchronize(D->stream));

  ss->embedding = D->x;
  ss->mha_q = D->q;
  ss->mha_att = D->att;
  ss->ffn_act = D->act;
  ss->logits = D->logits;
  ss->cached_count = 0;
  ss->k_cache = D->kc;  // device memory, bf16 elements when D->kv_bf16
  ss->v_cache = D->vc;
  ss->rope_cos_sin = D->rope;
  return t;
}

extern "C" void sg_free(transformer_t* t) {
  if (!t) return;
  Dev* D = t->device;
  if (D) {
    if (D->stream) HIP_CHECK(hipStreamSynchronize(D->stream));
    harvest(D);
    for (hipEvent_t e : D->event_pool) HIP_CHECK(hipEventDestroy(e));
    drop_graphs(D);
    for (int k = 0; k < W_COUNT; k++) {
      if (D->w[k] && !(k == W_OUT && D->tied)) HIP_CHECK(hipFree(D->w[k]));
    }
    void* bufs[] = {D->x, D->xn, D->q, D->att, D->act, D->kraw, D->logits, D->kc, D->vc,
                    D->rope, D->tok, D->pos, D->next, D->seq, D->seq_len, D->attn_part, D->attn_cnt,
                    D->gemv_part, D->gemv_cnt, D->am_v, D->am_i, D->cap_dev, D->cap_final_dev,
                    D->kp_hi, D->kp_lo, D->vt_hi, D->vt_lo,
                    D->moe_sel, D->moe_w, D->moe_act, D->moe_logits, D->moe_offs, D->moe_order, D->moe_out,
                    D->moe_ahi, D->moe_alo,
                    D->xn_hi, D->xn_lo,
                    D->att_hi, D->att_lo, D->act_hi, D->act_lo, D->ws, D->kstage};
    for (void* b : bufs)
      if (b) HIP_CHECK(hipFree(b));
    if (D->h_tok) HIP_CHECK(hipHostFree(D->h_tok));
    if (D->h_pos) HIP_CHECK(hipHostFree(D->h_pos));
    if (D->h_next) HIP_CHECK(hipHostFree(D->h_next));
    if (D->stream) HIP_CHECK(hipStreamDestroy(D->stream));
    delete D;
  }
  free(t->config->mrope_section);
  free(t->config);
  free(t->weights);
  free(t->state);
  free(t);
}

extern "C" void sg_print(FILE* f, const transformer_t* t) {
  if (!t) {
    fprintf(f, "transformer: NULL\n");
    return;
  }
  const transformer_configuration_t* c = t->config;
  fprintf(f, "Transformer (MI355X, %s):\n- Configuration:\n", sg_version());
  fprintf(f, "--- embedding_dim:      %zu\n", c->embedding_dim);
  fprintf(f, "--- head_dim:           %zu\n", c->head_dim);
  fprintf(f, "--- hidden_dim:         %zu\n", c->hidden_dim);
  fprintf(f, "--- layer_count:        %zu\n", c->layer_count);
  fprintf(f, "--- q_head_count:       %zu\n", c->q_head_count);
  fprintf(f, "--- kv_head_count:      %zu\n", c->kv_head_count);
  fprintf(f, "--- vocabulary_len:     %zu\n", c->vocabulary_len);
  fprintf(f, "--- context_len:        %zu\n", c->context_len);
  fprintf(f, "--- epsilon:            %g\n", c->epsilon);
  fprintf(f, "--- rope_theta:         %.1f\n", c->rope_theta);
  fprintf(f, "--- rope_pair_bound     %zu\n", c->rope_pair_bound);
  fprintf(f, "--- rope_pair_offset    %zu\n", c->rope_pair_offset);
  fprintf(f, "--- rope_pair_stride    %zu\n", c->rope_pair_stride);
  fprintf(f, "--- qk_norm:            %s\n", c->qk_norm ? "true" : "false");
  if (c->expert_count)
    fprintf(f, "--- experts:            %zu (top-%zu)\n", c->expert_count, c->expert_used_count);
  fprintf(f, "--- aliased_out_weight: %s\n", c->aliased_out_weight ? "true" : "false");
  fprintf(f, "- Weights (HBM):\n");
  const Dev* D = t->device;
  double total = 0, gb = 1024.0 * 1024.0 * 1024.0;
  for (int k = 0; k < W_COUNT; k++) {
    const Summary& sm = D->summary[k];
    if (!sm.present) continue;
    total += (double)sm.bytes;
    if (k >= W_GB) {
      fprintf(f, "--- %15s (%7.4f GB)\n", kClassName[k], sm.bytes / gb);
      continue;
    }
    fprintf(f, "--- %15s (%7.4f GB): [ %6.3f %6.3f %6.3f ... %6.3f %6.3f %6.3f ]\n",
            k == W_Q ? "mha_qkv" : kClassName[k], sm.bytes / gb, sm.first[0], sm.first[1],
            sm.first[2], sm.last[0], sm.last[1], sm.last[2]);
  }
  if (c->aliased_out_weight) fprintf(f, "--- %15s (%7.4f GB): alias to embedding\n", "out", 0.0);
  fprintf(f, "---  total size:%7.4f GB\n", total / gb);
}

extern "C" void sg_predict(transformer_t* t, size_t T, const int* token, size_t lc,
                           float* logits) {
  predict_device(t, T, token, lc, logits);
}

extern "C" int sg_predict_argmax(transformer_t* t, size_t T, const int* token) {
  Dev* D = t->device;
  predict_device(t, T, token, 1, nullptr);
  argmax_to(D, D->logits, false, false);
  HIP_CHECK(hipMemcpyAsync(D->h_next, D->next, sizeof(int), hipMemcpyDeviceToHost, D->stream));
  HIP_CHECK(hipStreamSynchronize(D->stream));
  return *D->h_next;
}

extern "C" size_t sg_generate_greedy(transformer_t* t, size_t T, const int* token,
                                     size_t steps, int eos, int* out,
                                     transformer_timing_t* timing) {
  Dev* D = t->device;
  if (T == 0 || steps == 0) ST_DIE("transformer_generate_greedy: needs tokens and steps");
  if (t->state->cached_count + T + (steps - 1) > (size_t)D->ctx)
    ST_DIE("context length exhausted");
  HIP_CHECK(hipMemsetAsync(D->seq_len, 0, sizeof(int), D->stream));
  HIP_CHECK(hipStreamSynchronize(D->stream));
  const double t0 = now_s();
  predict_device(t, T, token, 1, nullptr);
  argmax_to(D, D->logits, true, false);
  HIP_CHECK(hipStreamSynchronize(D->stream));
  harvest(D);
  const double t1 = now_s();
  // The token predicted from the prompt never ends the loop: the reference
  // tests only the decode steps' tokens against EOS (source/strasgpt.c:
  // 217-248).
  size_t produced = 1;
  bool stop = false;
  if (steps > 1) {
    const bool eager = D->prof || !D->use_graph || D->decode_mode == TRANSFORMER_DECODE_EAGER;
    if (!eager) build_decode_graph(D);
    set_pos(D, t->state->cached_count);
    for (size_t i = 1; i < steps && !stop; i++) {
      if (eager) {
        // Eager step (events around every launch); same kernels as the graph.
        D->host_pos = t->state->cached_count + produced - 1;
        forward_chunk(D, D->next, 1, 1);
        argmax_to(D, D->logits, true, true);
        HIP_CHECK(hipStreamSynchronize(D->stream));
        harvest(D);
      } else {
        HIP_CHECK(hipGraphLaunch(D->graph, D->stream));
      }
      produced++;
      if (eos >= 0) {
        HIP_CHECK(hipMemcpyAsync(D->h_next, D->next, sizeof(int), hipMemcpyDeviceToHost, D->stream));
        HIP_CHECK(hipStreamSynchronize(D->stream));
        stop = *D->h_next == eos;
      }
    }
    HIP_CHECK(hipStreamSynchronize(D->stream));
    t->state->cached_count += produced - 1;
  }
  const double t2 = now_s();
  HIP_CHECK(hipMemcpy(out, D->seq, produced * sizeof(int), hipMemcpyDeviceToHost));
  if (timing) {
    timing->prefill_s = t1 - t0;
    timing->decode_s = t2 - t1;
    timing->decode_count = produced - 1;
  }
  return produced;
}

extern "C" size_t sg_generate_sampled(transformer_t* t, size_t T, const int* token, size_t steps,
                                      int eos, sampler_hip* smp, int* out, transformer_timing_t* timing) {
  Dev* D = t->device;
  if (!smp) ST_DIE("transformer_generate_sampled: NULL sampler");
  if (smp->V != D->V) ST_DIE("transformer_generate_sampled: sampler vocabulary differs from the model's");
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  if (dev != smp->device) ST_DIE("transformer_generate_sampled: sampler built on another device");
  if (T == 0 || steps == 0) ST_DIE("transformer_generate_sampled: needs tokens and steps");
  if (t->state->cached_count + T + (steps - 1) > (size_t)D->ctx) ST_DIE("context length exhausted");
  HIP_CHECK(hipStreamSynchronize(smp->stream));  // earlier host-array draws are done
  HIP_CHECK(hipMemsetAsync(D->seq_len, 0, sizeof(int), D->stream));
  HIP_CHECK(hipStreamSynchronize(D->stream));
  const double t0 = now_s();
  predict_device(t, T, token, 1, nullptr);
  sg::sample(sampler_params(smp, D->logits, nullptr, token[T - 1], D->next, D->seq, D->seq_len, nullptr),
             D->stream);
  HIP_CHECK(hipStreamSynchronize(D->stream));
  harvest(D);
  const double t1 = now_s();
  // The token predicted from the prompt never ends the loop: the reference
  // tests only the decode steps' tokens against EOS (source/strasgpt.c:
  // 217-248).
  size_t produced = 1;
  bool stop = false;
  if (steps > 1) {
    const bool eager = D->prof || !D->use_graph || D->decode_mode == TRANSFORMER_DECODE_EAGER;
    if (!eager) build_decode_graph(D, false);
    set_pos(D, t->state->cached_count);
    for (size_t i = 1; i < steps && !stop; i++) {
      if (eager) {
        D->host_pos = t->state->cached_count + produced - 1;
        forward_chunk(D, D->next, 1, 1);
      } else {
        HIP_CHECK(hipGraphLaunch(D->graph_body, D->stream));
      }
      // the previous token (the one just fed) is read before the draw overwrites it
      sg::sample(sampler_params(smp, D->logits, D->next, -1, D->next, D->seq, D->seq_len, D->pos), D->stream);
      if (eager) {
        HIP_CHECK(hipStreamSynchronize(D->stream));
        harvest(D);
      }
      produced++;
      if (eos >= 0) {
        HIP_CHECK(hipMemcpyAsync(D->h_next, D->next, sizeof(int), hipMemcpyDeviceToHost, D->stream));
        HIP_CHECK(hipStreamSynchronize(D->stream));
        stop = *D->h_next == eos;
      }
    }
    HIP_CHECK(hipStreamSynchronize(D->stream));
    t->state->cached_count += produced - 1;
  }
  const double t2 = now_s();
  HIP_CHECK(hipMemcpy(out, D->seq, produced * sizeof(int), hipMemcpyDeviceToHost));
  if (timing) {
    timing->prefill_s = t1 - t0;
    timing->decode_s = t2 - t1;
    timing->decode_count = produced - 1;
  }
  return produced;
}

// The bf16 planes of the cache hold rows [0, cached_count) of the current
// sequence (prefill chunks and decode steps write them).
extern "C" void sg_reset(transformer_t* t) {
  t->state->cached_count = 0;
}

extern "C" void sg_capture_hidden(transformer_t* t, float* out, float* out_final) {
  Dev* D = t->device;
  if (!out || !out_final) {
    D->cap_out = nullptr;
    D->cap_final = nullptr;
    return;
  }
  if (!D->cap_dev) {
    D->cap_dev = dalloc<float>((size_t)D->L * TRANSFORMER_CHUNK_MAX_LEN * D->d);
    D->cap_final_dev = dalloc<float>((size_t)TRANSFORMER_CHUNK_MAX_LEN * D->d);
  }
  D->cap_out = out;
  D->cap_final = out_final;
}

extern "C" int sg_set_prefill_precision(transformer_t* t, int mode) {
  if (mode != sg::GEMM_SPLIT2 && mode != sg::GEMM_BF16) ST_DIE("unknown prefill precision");
  const int old = t->device->precision;
  t->device->precision = mode;
  return old;
}

extern "C" int sg_set_kv_cache_format(transformer_t* t, int format) {
  if (format != TRANSFORMER_KV_FP32 && format != TRANSFORMER_KV_BF16) ST_DIE("unknown KV-cache format");
  Dev* D = t->device;
  if (t->state->cached_count != 0)
    ST_DIE("the KV-cache format can only change while the cache is empty (before the first token or "
           "after transformer_reset)");
  const int old = D->kv_bf16 ? TRANSFORMER_KV_BF16 : TRANSFORMER_KV_FP32;
  if (format == old) return old;
  HIP_CHECK(hipStreamSynchronize(D->stream));
  if (D->graph || D->graph_body) {  // the captured decode step points at the old cache
    drop_graphs(D);
  }
  HIP_CHECK(hipFree(D->kc));
  HIP_CHECK(hipFree(D->vc));
  if (D->kstage) HIP_CHECK(hipFree(D->kstage));
  D->kc = D->vc = D->kstage = nullptr;
  D->kv_bf16 = format == TRANSFORMER_KV_BF16;
  alloc_kv(D, (size_t)D->L * D->kvh * D->ctx * D->hd);
  t->state->k_cache = D->kc;
  t->state->v_cache = D->vc;
  HIP_CHECK(hipStreamSynchronize(D->stream));
  return old;
}

extern "C" int sg_set_decode_mode(transformer_t* t, int mode) {
  if (mode != TRANSFORMER_DECODE_GRAPH && mode != TRANSFORMER_DECODE_EAGER)
    ST_DIE("unknown decode mode");
  Dev* D = t->device;
  HIP_CHECK(hipStreamSynchronize(D->stream));
  const int old = D->decode_mode;
  D->decode_mode = mode;
  return old;
}

extern "C" void sg_profile(transformer_t* t, int enable) {
  Dev* D = t->device;
  HIP_CHECK(hipStreamSynchronize(D->stream));
  harvest(D);
  if (enable) memset(D->stat, 0, sizeof(D->stat));
  D->prof = enable != 0;
}

extern "C" int sg_kernel_rate(transformer_t* t, int cls, int reps, double* avg_us, double* bytes) {
  Dev* D = t->device;
  const bool dense = cls == K_GU_GEMV && !D->moe, moe = cls == K_MOE_GU && D->moe;
  if (!(dense || moe) || reps <= 0) return -1;
  hipStream_t s = D->stream;
  const double d = D->d;
  // MoE: the decode launch of one token, experts from the router logits (or
  // selection) left by the last step, the same for every layer; each
  // layer's experts are its own weights, so every launch streams from HBM.
  const bool fused = sg::moe_route_logits_supported(D->E, D->topk, D->d);
  if (moe && !fused) return -1;  // the selection buffer may not hold valid expert ids yet
  auto launch = [&](int l) {
    if (moe) {
      sg::MoeGemvParams g{};
      g.blocks = W8(D, W_GB, l);
      g.scales = W8(D, W_GS, l);
      g.blocks2 = W8(D, W_UB, l);
      g.scales2 = W8(D, W_US, l);
      g.x = D->xn;
      g.logits = D->moe_logits;  // top-k in the kernel: ids always in [0, E)
      g.E = D->E;
      g.tokens = 1;
      g.topk = D->topk;
      g.N = D->H;
      g.K = D->d;
      g.y = D->moe_act;  // scratch: the generation state is untouched
      sg::moe_gemv_swiglu(g, s);
      return;
    }
    sg::GemvParams f{};
    f.w = W16(D, W_GATE, l);
    f.w2 = W16(D, W_UP, l);
    f.x = D->x;
    f.norm_w = W16(D, W_FFN_NORM, l);
    f.eps = D->eps;
    f.N = D->H;
    f.K = D->d;
    f.y = D->act;  // scratch: the generation state is untouched
    sg::gemv(f, sg::GEMV_SWIGLU, s);
  };
  HIP_CHECK(hipStreamSynchronize(s));
  for (int l = 0; l < D->L; l++) launch(l);  // warm the code path
  hipEvent_t a, b;
  HIP_CHECK(hipEventCreate(&a));
  HIP_CHECK(hipEventCreate(&b));
  HIP_CHECK(hipEventRecord(a, s));
  for (int r = 0; r < reps; r++)
    for (int l = 0; l < D->L; l++) launch(l);
  HIP_CHECK(hipEventRecord(b, s));
  HIP_CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  HIP_CHECK(hipEventElapsedTime(&ms, a, b));
  HIP_CHECK(hipEventDestroy(a));
  HIP_CHECK(hipEventDestroy(b));
  *avg_us = ms * 1e3 / ((double)reps * D->L);
  *bytes = moe ? D->topk * mxfp4_bytes(2.0 * D->H * d) : 2.0 * D->H * d * 2;
  return 0;
}

extern "C" int sg_profile_read(transformer_t* t, int cls, transformer_kernel_stat_t* out) {
  if (cls < 0 || cls >= TRANSFORMER_K_CLASS_COUNT) return -1;
  *out = t->device->stat[cls];
  return 0;
}

extern "C" const char* sg_version(void) {
  return "strasgpt-hip gfx950 (decode GEMV bf16/MXFP4 -> fp32; prefill GEMM MFMA 32x32x16 and 16x16x32 "
         "bf16x2; split-bf16 MFMA attention)";
}
