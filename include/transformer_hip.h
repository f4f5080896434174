/*
 * Extensions of the StrasGPT C API that have no single reference entry
 * point. Each one names the reference code it stands in for.
 */
#ifndef TRANSFORMER_HIP_H
# define TRANSFORMER_HIP_H

#include "transformer.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Greedy next-token selection on the device: transformer_predict with
 * logits_count = 1 followed by the reference's sample_argmax (first index
 * of the maximum, reference source/sampler.c:92-102) without copying the
 * logits to the host. Returns the token id. */
int transformer_predict_argmax(
    transformer_t* transformer, size_t token_count, const int* token
);

typedef struct transformer_timing {
  double prefill_s; /* first transformer_predict over the prompt */
  double decode_s;  /* sum of the single-token steps */
  size_t decode_count;
} transformer_timing_t;

/* The reference driver's greedy loop (source/strasgpt.c:206-252 with
 * --temp 0): one prefill over the prompt, then step_count - 1 single-token
 * steps, each feeding back the argmax. The loop stays on the device: the
 * next token never leaves HBM between steps. By default the step's
 * kernels are replayed from a captured HIP graph (see
 * transformer_set_decode_mode). Writes step_count token ids to out. Stops
 * early, like the reference, when a decode step produces eos_token_id >= 0
 * (the token predicted from the prompt is not tested, as in
 * source/strasgpt.c:217-248); returns the number of ids written. timing may be NULL. Environment:
 * STRASGPT_DECODE_GRAPH=0 launches the step's kernels eagerly instead (for
 * tools that do not follow graph launches). */
size_t transformer_generate_greedy(
    transformer_t* transformer,
    size_t token_count,
    const int* token,
    size_t step_count,
    int eos_token_id,
    int* out,
    transformer_timing_t* timing
);

/* transformer_generate_greedy with the reference's stochastic sampler in
 * place of the argmax (source/strasgpt.c:206-252 with sampler_sample,
 * source/sampler.c:234-337), every draw on the device: after the prompt,
 * the sampler draws from the last row's logits with the prompt's last
 * token as the previous token; each decode step feeds the drawn token and
 * draws again with it as the previous token. The sampler (sampler_hip.h)
 * carries the parameters, the generator state and the presence marks
 * across calls, as the reference's sampler_t does; it must have the
 * model's vocabulary and live on the same device. A temperature of 0 gives
 * transformer_generate_greedy's tokens. */
struct sampler_hip;
size_t transformer_generate_sampled(
    transformer_t* transformer,
    size_t token_count,
    const int* token,
    size_t step_count,
    int eos_token_id,
    struct sampler_hip* sampler,
    int* out,
    transformer_timing_t* timing
);

/* Forget the KV cache (cached_count = 0) so that one loaded model can
 * serve another sequence. The reference has no reset: it builds a new
 * transformer_t per sequence. */
void transformer_reset(transformer_t* transformer);

/* Parity hook: when out is not NULL, the next transformer_predict copies
 * the residual stream after every layer into out as
 * [layer_count][token_count][embedding_dim] fp32 (the reference's
 * embedding[t][e] after source/transformer.c:1498-1504), and the
 * final-RMSNorm output into out_final as [token_count][embedding_dim]
 * (source/transformer.c:1580-1590). The hook covers one call of at most
 * TRANSFORMER_CHUNK_MAX_LEN tokens and is then cleared. */
void transformer_capture_hidden(
    transformer_t* transformer, float* out, float* out_final
);

/* GEMM arithmetic for prefill chunks longer than the GEMV threshold.
 * 0: bf16x2 (fp32 activations split into two bf16 terms; products exact,
 *    fp32 accumulate: matches the fp32 reference to fp32 rounding noise),
 * 1: bf16 (activations rounded once to bf16: twice the MFMA rate, logits
 *    move by about 1e-3 so greedy tokens can differ from the reference).
 * Returns the previous mode. */
int transformer_set_prefill_precision(transformer_t* transformer, int mode);

/* Decode step implementation used by transformer_generate_greedy (no
 * reference counterpart): one kernel per operation, either
 *   TRANSFORMER_DECODE_GRAPH (default): replayed from a captured HIP graph,
 *   TRANSFORMER_DECODE_EAGER: launched one by one.
 * Returns the previous mode. Profiling (transformer_profile) always uses
 * the eager path. */
enum transformer_decode_mode {
  TRANSFORMER_DECODE_GRAPH = 1,
  TRANSFORMER_DECODE_EAGER = 2
};
int transformer_set_decode_mode(transformer_t* transformer, int mode);

/* KV-cache storage format (no reference counterpart: the reference cache
 * is fp32, include/transformer.h:76-77, written at
 * source/transformer.c:1271-1291). TRANSFORMER_KV_BF16 stores every key
 * (after its norm and RoPE) and value rounded to the nearest bf16, in the
 * same [layer][kv_head][position][head_dim] layout: half the cache memory
 * and half the bytes decode attention reads. Attention reads the stored
 * values exactly, so results differ from the fp32 cache by that rounding
 * only. The initial format is fp32, or bf16 when the environment variable
 * STRASGPT_KV_CACHE=bf16 is set at load time. The format can change only
 * while the cache is empty (before the first token or right after
 * transformer_reset); it dies otherwise. Returns the previous format. The
 * fp32 prefill attention kernel (STRASGPT_PREFILL_ATTN=fp32) needs the fp32
 * cache. */
enum transformer_kv_format {
  TRANSFORMER_KV_FP32 = 0,
  TRANSFORMER_KV_BF16 = 1
};
int transformer_set_kv_cache_format(transformer_t* transformer, int format);

/* Measurement hooks (no reference counterpart; the reference only times
 * whole predict calls, source/strasgpt.c:206-274). While enabled, every
 * kernel launch of the forward pass is bracketed by HIP events on the
 * library's stream and the decode loop of transformer_generate_greedy runs
 * eagerly instead of replaying its graph. Statistics accumulate per kernel
 * class until profiling is enabled again (which clears them). Algorithmic
 * bytes and FLOP are the work the kernel's inputs define, not counters. */
enum transformer_kernel_class {
  TRANSFORMER_K_QKV_GEMV, TRANSFORMER_K_ATTENTION_DECODE, TRANSFORMER_K_O_GEMV,
  TRANSFORMER_K_GATE_UP_GEMV, TRANSFORMER_K_DOWN_GEMV, TRANSFORMER_K_LOGITS_GEMV,
  TRANSFORMER_K_ARGMAX, TRANSFORMER_K_MOE_ROUTE, TRANSFORMER_K_MOE_GATE_UP,
  TRANSFORMER_K_MOE_DOWN, TRANSFORMER_K_QKV_GEMM, TRANSFORMER_K_ATTENTION_PREFILL,
  TRANSFORMER_K_O_GEMM, TRANSFORMER_K_GATE_UP_GEMM, TRANSFORMER_K_DOWN_GEMM,
  TRANSFORMER_K_ELEMENTWISE,
  /* MoE FFN of prompt chunks (more than one token): router, expert
   * gate/up + SwiGLU and down projections (grouped MFMA GEMMs from 8
   * tokens on); the MOE classes above count single-token decode steps. */
  TRANSFORMER_K_MOE_ROUTE_PREFILL, TRANSFORMER_K_MOE_GATE_UP_PREFILL,
  TRANSFORMER_K_MOE_DOWN_PREFILL, TRANSFORMER_K_CLASS_COUNT
};

typedef struct transformer_kernel_stat {
  size_t launches;
  double total_ms; /* sum of event-measured launch durations */
  double bytes;    /* algorithmic HBM bytes, summed over launches */
  double flops;    /* algorithmic FLOP, summed over launches */
} transformer_kernel_stat_t;

void transformer_profile(transformer_t* transformer, int enable);
/* Returns 0, or -1 for an unknown kernel class. */
int transformer_profile_read(
    transformer_t* transformer, int kernel_class, transformer_kernel_stat_t* out
);

/* Sustained rate of one decode kernel class: `reps` passes of back-to-back
 * launches over every layer's weights (same shapes and inputs as a decode
 * step), bracketed by one pair of events on the library's stream. Writes
 * the average duration per launch (one inter-kernel gap included, as in a
 * decode step) and the algorithmic bytes per launch. Supported for the
 * dense gate/up GEMV (TRANSFORMER_K_GATE_UP_GEMV) and the MoE expert
 * gate/up GEMV (TRANSFORMER_K_MOE_GATE_UP; the experts that the router
 * logits of the last decode step select, the same for every layer, or
 * experts 0 .. top-k - 1 before any decode step), whose launches write only
 * scratch activations; returns -1 for other classes. No reference
 * counterpart (measurement hook). */
int transformer_kernel_rate(
    transformer_t* transformer, int kernel_class, int reps, double* avg_us,
    double* bytes_per_launch
);

/* Library build identification (gfx target, kernel variants). */
const char* transformer_hip_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TRANSFORMER_HIP_H */
