/*
 * hfmoe.h -- C-ABI of the MI355X (gfx950) MoE-block library, libhfmoe.so.
 *
 * Drop-in boundary for HummingFlight's MoE block.  The engine keeps
 * GLMForward::moeLayer(int layer, const float* input, float* output)
 * (src/model/glm_forward.h:93) and its weight handles (TensorLocation /
 * ExpertWeights / LayerWeights, src/model/weight_index.h:14-68) and calls
 * these entry points; the per-expert GPU plugin surface of
 * src/compute/cuda_backend.h:23-90 is covered one for one.
 *
 * Conventions (cuda_backend.h:56-62 uses bool; here):
 *   - every entry point returns an int status, HFMOE_OK (0) on success; the
 *     engine shim maps a non-zero status to the reference's `false`, which
 *     makes moeLayer restart the layer on its own CPU path
 *     (glm_forward.cpp:594-602).  The library itself has no CPU compute path.
 *   - hfmoe_last_error() describes the most recent failure.
 *   - no C++ exceptions cross this boundary; no torch types appear in it.
 *   - pointers named *_dev are HBM addresses; *_host are host addresses.
 *   - not thread-safe: one caller thread, as the reference's generation
 *     thread (cuda_backend.cpp:366 is a process-global singleton too).
 *   - `stream` arguments are hipStream_t values; NULL selects the library's
 *     own stream (default priority).
 */
#ifndef HFMOE_H
#define HFMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HFMOE_OK = 0,
    HFMOE_ERR_NO_DEVICE = 1,
    HFMOE_ERR_NOT_INITIALIZED = 2,
    HFMOE_ERR_INVALID_ARGUMENT = 3,
    HFMOE_ERR_UNSUPPORTED = 4,
    HFMOE_ERR_OUT_OF_MEMORY = 5,
    HFMOE_ERR_NOT_REGISTERED = 6,
    HFMOE_ERR_HIP = 7
};

/* Where a layer's routed-expert weights live. */
enum {
    HFMOE_EXPERTS_DEVICE = 0,      /* HBM-resident, read in place */
    HFMOE_EXPERTS_HOST_PINNED = 1  /* pinned host RAM; only selected experts are
                                      copied to HBM (hipMemcpyAsync, side stream) */
};

/* MoE fields of ModelConfig (src/model/config.h:49-58,78) plus budgets. */
typedef struct hfmoe_config {
    int32_t hidden;               /* hiddenSize */
    int32_t moe_intermediate;     /* moeIntermediateSize (one routed expert) */
    int32_t n_routed_experts;     /* numLocalExperts, <= 1024 */
    int32_t num_experts_per_tok;  /* numExpertsPerTok, 1..8 */
    int32_t n_group;              /* 1 = flat noaux_tc (the reference's rule) */
    int32_t topk_group;           /* groups kept when n_group > 1 (config.h:58) */
    int32_t n_shared_experts;     /* nSharedExperts; shared inter = n * moe_intermediate */
    int32_t norm_topk_prob;       /* normTopkProb */
    float routed_scaling_factor;  /* routedScalingFactor */
    float rms_norm_eps;           /* rmsNormEps */
    uint64_t vram_budget_bytes;   /* AdaptiveConfig::vramBudgetBytes
                                     (src/runtime/runtime_config.h:62); bounds the
                                     streamed-expert staging pool; 0 = default */
    int32_t max_tokens;           /* largest T of one forward call (workspace), <= 8192 */
    int32_t reserved;
} hfmoe_config;

/* One MoE layer's tensors (LayerWeights / ExpertWeights,
 * src/model/weight_index.h:28-36,58-67).  BF16 values are raw uint16 bits. */
/* Alignment: BF16 matrices read from HBM (router, shared expert, routed
 * experts with HFMOE_EXPERTS_DEVICE) must be 16-byte aligned, the bias 4-byte
 * and the norm weight 2-byte; hfmoe_register_layer returns
 * HFMOE_ERR_INVALID_ARGUMENT otherwise.  Host-pinned experts may sit at any
 * address (the DMA engines copy them into the library's aligned slots). */
typedef struct hfmoe_layer_weights {
    const uint16_t* router_dev;       /* mlp.gate.weight      [E, hidden] */
    const float* score_bias_dev;      /* e_score_correction_bias F32 [E], or NULL */
    const uint16_t* shared_gate_dev;  /* shared_experts.gate_proj [S*I, hidden] */
    const uint16_t* shared_up_dev;    /* shared_experts.up_proj   [S*I, hidden] */
    const uint16_t* shared_down_dev;  /* shared_experts.down_proj [hidden, S*I] */
    const uint16_t* const* experts;   /* host array of 3*E pointers, expert e at
                                         [3e] gate [I,hidden], [3e+1] up [I,hidden],
                                         [3e+2] down [hidden,I]; HBM or pinned host
                                         addresses per experts_location */
    const uint16_t* post_attention_norm_dev; /* RMSNorm weight BF16 [hidden] or NULL
                                                (used by hfmoe_mlp_block) */
    int32_t experts_location;         /* HFMOE_EXPERTS_* */
    int32_t reserved;
} hfmoe_layer_weights;

/* Optional routing outputs of a forward call (HBM pointers, any may be NULL). */
typedef struct hfmoe_route_debug {
    float* logits_dev;     /* [T, E] router GEMV before sigmoid */
    int32_t* idx_dev;      /* [T, k] selected experts, descending biased score */
    float* weight_dev;     /* [T, k] normalised, scaled routing weights */
    int32_t* offsets_dev;  /* [E+1] dispatch offsets (T > 1 paths) */
    int32_t* perm_dev;     /* [T*k] pair ids t*k+r ordered by (expert, pair) */
} hfmoe_route_debug;

/* ---- device lifetime (cuda_backend.h:23-34) ---- */
int hfmoe_init(int device);                      /* cudaInit */
void hfmoe_shutdown(void);                       /* cudaShutdown */
int hfmoe_available(void);                       /* gpuAvailable: 1 after init */
int hfmoe_device_name(char* buf, size_t len);    /* cudaDeviceName */
size_t hfmoe_device_memory_mb(void);             /* cudaDeviceMemoryMB */
const char* hfmoe_last_error(void);

/* ---- MoE layer (GLMForward::moeLayer, glm_forward.h:93) ---- */
int hfmoe_configure(const hfmoe_config* cfg);
int hfmoe_register_layer(int layer, const hfmoe_layer_weights* w);
/* out_dev[T, hidden] = MoE(x_dev[T, hidden]), FP32 in and out, device pointers. */
int hfmoe_moe_forward(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream);
int hfmoe_moe_forward_debug(int layer, const float* x_dev, int32_t T, float* out_dev,
                            void* stream, const hfmoe_route_debug* dbg);
/* hfmoe_moe_forward for one token (T <= 1) that allocates nothing: no
 * counterpart in the reference; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Its scratch (router logits, score pairs, selection, h) lives in
 * a 192 KiB static device array per GPU, held until the process ends; every
 * shape hfmoe_configure accepts fits.  HBM-resident MoE layers only.  Calls on
 * one GPU share that array: calls that overlap in time on one GPU race. */
int hfmoe_moe_forward_noalloc(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream);
/* hfmoe_moe_forward with the activations as BF16 bits [T, hidden] (16-byte
 * aligned): moeLayer's FP32 input (glm_forward.h:93) held as BF16 by an engine
 * that keeps its activations in BF16.  x is widened to FP32 exactly, into the
 * library's scratch rows, and the FP32 forward runs on the same stream: the
 * output equals hfmoe_moe_forward's on those FP32 values, bit for bit. */
int hfmoe_moe_forward_bf16(int layer, const uint16_t* x_dev, int32_t T, float* out_dev, void* stream);
/* The moeLayer contract itself: one token, host FP32 buffers, synchronous. */
int hfmoe_moe_layer(int layer, const float* input_host, float* output_host);
/* h_dev[T, hidden] += MLP(RMSNorm(h_dev)) -- the MLP half of a decoder layer
 * (glm_forward.cpp:785-796): the MoE block, or the dense MLP for a layer
 * registered with hfmoe_register_dense_layer.  h_dev 16-byte aligned; T = 0
 * does nothing. */
int hfmoe_mlp_block(int layer, float* h_dev, int32_t T, void* stream);

/* ---- dense MLP layers (the first first_k_dense_replace layers, config.h:53;
 *      GLMForward::denseMlp, glm_forward.cpp:410-432) ---- */
typedef struct hfmoe_dense_weights {
    const uint16_t* gate_dev;  /* mlp.gate_proj.weight [inter, hidden] BF16 */
    const uint16_t* up_dev;    /* mlp.up_proj.weight   [inter, hidden] */
    const uint16_t* down_dev;  /* mlp.down_proj.weight [hidden, inter] */
    const uint16_t* post_attention_norm_dev;  /* [hidden] or NULL (hfmoe_mlp_block) */
    int32_t intermediate;      /* intermediateSize (config.h:16) */
    int32_t reserved;
} hfmoe_dense_weights;
/* The three matrices must be 16-byte aligned, the norm weight 2-byte. */
int hfmoe_register_dense_layer(int layer, const hfmoe_dense_weights* w);
/* out_dev[T, hidden] = Wd.(silu(Wg.x) * (Wu.x)), FP32 in and out. */
int hfmoe_dense_mlp_forward(int layer, const float* x_dev, int32_t T, float* out_dev, void* stream);

/* ---- LM head (GLMForward::lmHeadAndSample, glm_forward.cpp:663-731) ---- */
/* lm_head.weight [vocab, hidden] BF16 and model.norm.weight [hidden] (NULL:
 * ones), both caller-owned HBM; replaces any earlier registration. */
int hfmoe_register_lm_head(const uint16_t* lm_head_dev, const uint16_t* final_norm_dev, int32_t vocab);
/* logits_dev[T, vocab] = lm_head . RMSNorm(h_dev[t]); token_dev[t] (optional)
 * = first index of the largest logit (greedy sampling). */
int hfmoe_lm_head(const float* h_dev, int32_t T, float* logits_dev, int32_t* token_dev, void* stream);

/* ---- plugin helpers (cuda_backend.h:36-48): host buffers, synchronous ---- */
int hfmoe_embedding_lookup(const uint16_t* emb_host, int token_id, float* out_host, int hidden); /* gpuEmbeddingLookup */
int hfmoe_matvec_bf16(const uint16_t* w_host, const float* x_host, float* y_host, int M, int K);  /* gpuMatvecBf16 */
int hfmoe_softmax(float* x_host, int n);                                                          /* gpuSoftmax */
int hfmoe_argmax(const float* x_host, int n, int32_t* best);                                       /* gpuArgmax */
/* Device forms, queued on `stream` (glm_cuda::embeddingGather / matvec /
 * softmax / argmax, cuda_kernels.h:8-11).  hfmoe_embedding: out_dev[t, :] =
 * emb_dev[ids_dev[t], :] as FP32, ids outside [0, vocab) give zeros;
 * hfmoe_embedding_gather: one row, token_id < vocab is the caller's to check
 * (as in the reference); softmax / argmax: each of T rows of n (argmax: the
 * first largest element, an int32 per row). */
int hfmoe_embedding(const uint16_t* emb_dev, int32_t vocab, int32_t hidden, const int32_t* ids_dev, int32_t T,
                    float* out_dev, void* stream);
int hfmoe_embedding_gather(const uint16_t* emb_dev, int token_id, float* out_dev, int hidden, void* stream);
int hfmoe_matvec_bf16_dev(const uint16_t* w_dev, const float* x_dev, float* y_dev, int M, int K, void* stream);
int hfmoe_softmax_rows(float* x_dev, int32_t T, int32_t n, void* stream);
int hfmoe_argmax_rows(const float* x_dev, int32_t T, int32_t n, int32_t* best_dev, void* stream);
/* y_dev[i] = 1 / (1 + expf(-x_dev[i])) in float, i < n: the router's scoring
 * function (sigmoid_f32, moe_router.h:19-21), bit-identical to the reference's
 * (glibc's expf) for every float input. */
int hfmoe_router_sigmoid(const float* x_dev, float* y_dev, int64_t n, void* stream);

/* ---- per-expert plugin surface (cuda_backend.h:64-90) ---- */
int hfmoe_expert_cache_config(int capacity, int staging_depth); /* gpuExpertCacheConfig */
void hfmoe_expert_cache_shutdown(void);                         /* gpuExpertCacheShutdown */
int hfmoe_experts_enabled(void);                                /* gpuExpertsEnabled */
int hfmoe_expert_stage(int layer, int expert_id, const uint16_t* w_host, int hidden,
                       int inter);                              /* gpuExpertStage */
int hfmoe_expert_ffn(int layer, int expert_id, const float* x_host, float* out_host,
                     int hidden, int inter);                    /* gpuExpertFFN */
int hfmoe_self_test(void);                                      /* cudaExpertSelfTest */

/* ---- buffers and synthetic data (no counterpart: harness plumbing) ---- */
int hfmoe_malloc(void** ptr_dev, size_t bytes);
int hfmoe_free(void* ptr_dev);
int hfmoe_host_alloc(void** ptr_host, size_t bytes);   /* pinned host memory */
int hfmoe_host_free(void* ptr_host);
int hfmoe_memcpy_h2d(void* dst_dev, const void* src_host, size_t bytes);
int hfmoe_memcpy_d2h(void* dst_host, const void* src_dev, size_t bytes);
int hfmoe_memcpy_d2d(void* dst_dev, const void* src_dev, size_t bytes);
int hfmoe_memset(void* ptr_dev, int value, size_t bytes);
int hfmoe_synchronize(void);
/* Seeded counter-based N(mean, std) tensors in HBM (BF16 bits or F32). */
int hfmoe_fill_normal_bf16(uint16_t* dst_dev, uint64_t n, uint64_t seed, uint64_t tensor,
                           uint64_t first, float mean, float std);
int hfmoe_fill_normal_f32(float* dst_dev, uint64_t n, uint64_t seed, uint64_t tensor,
                          uint64_t first, float mean, float std);

/* ---- streamed experts: HBM expert cache and next-layer copy-ahead ----
 * Layers registered with HFMOE_EXPERTS_HOST_PINNED copy their selected
 * experts into an LRU pool of HBM slots (ExpertGpuCache, cuda_backend.cpp:
 * 196-363; size from vram_budget_bytes).  Once a layer has routed, the experts
 * predicted for the next layer -- the previous token's selection there -- are
 * copied ahead while the layer computes (Scheduler::onLayerRouterDone /
 * predictNextLayerExperts, src/engine/scheduler.cpp:180-219,238-388), unless
 * that layer's winner-overlap EMA is below overlap_floor. */
typedef struct hfmoe_stream_options {
    int32_t prefetch_next_layer;  /* 1 (default): copy predicted next-layer experts ahead */
    int32_t ema_predictor;        /* setPopularityPredictor(alpha, enable)
                                     (scheduler.cpp:158-165); default 0 */
    float ema_alpha;              /* heat blend, (0, 1]; default 0.1 */
    float overlap_floor;          /* kSpecOverlapFloor (scheduler.cpp:51), default 0.5 */
    float overlap_alpha;          /* kSpecOverlapAlpha (scheduler.cpp:52), default 0.5 */
    /* Router-probability mode, Scheduler::setRouterPrefetch(prefetchExtraDepth,
     * probPriority) (scheduler.cpp:148-156, rules :320-352); both off by default. */
    int32_t extra_depth;          /* copy ahead this many more of the token's winners, by
                                     descending routing weight, as next-layer guesses */
    int32_t prob_resident;        /* 1: pin a resident winner whose routing weight is >= 0.9 x
                                     the layer's running maximum once looked up twice before */
    int32_t reserved;
} hfmoe_stream_options;

/* InferenceStats routedPredStaged / routedPredConsumed / prefetchWasted
 * (src/engine/inference_stats.h:25-35) and the cache's hit counts. */
typedef struct hfmoe_stream_counters {
    uint64_t lookups;        /* selected experts looked up */
    uint64_t hits;           /* ... resident or already being copied ahead */
    uint64_t misses;         /* ... copied on demand */
    uint64_t pred_staged;    /* predicted experts copied ahead */
    uint64_t pred_consumed;  /* copied-ahead experts a lookup then used */
    uint64_t pred_wasted;    /* copied-ahead experts evicted unused */
    uint64_t pred_resident;  /* predictions already resident (no copy) */
    uint64_t copies;         /* expert weight sets copied host -> HBM */
    int32_t slots;           /* HBM slots in the pool (0 before the first streamed call) */
    int32_t pinned;          /* resident experts pinned by prob_resident (saturates at INT32_MAX) */
} hfmoe_stream_counters;     /* 72 bytes: pinned sits in what was the reserved field, so the
                                layout and size are those of the first published header */
#ifdef __cplusplus
static_assert(sizeof(hfmoe_stream_counters) == 72, "hfmoe_stream_counters layout");
#else
_Static_assert(sizeof(hfmoe_stream_counters) == 72, "hfmoe_stream_counters layout");
#endif

int hfmoe_stream_set_options(const hfmoe_stream_options* opt);
int hfmoe_stream_get_options(hfmoe_stream_options* opt);
int hfmoe_stream_read_counters(hfmoe_stream_counters* out);
int hfmoe_stream_reset(void);  /* empty the pool, forget routing history, zero counters */

/* ---- checkpoints: safetensors shards -> registered MoE layers ----
 * WeightIndex::build (src/model/weight_index.cpp:84-266) over strict shard
 * parsing (SafeTensorsFile::open with strictStOpts, safetensors.cpp:60-240,
 * weight_index.cpp:20-27): BF16 only, F32 allowed for
 * "e_score_correction_bias"; rejected tensors are counted and skipped. */
typedef struct hfmoe_checkpoint hfmoe_checkpoint;  /* opaque */

typedef struct hfmoe_safetensors_stats {  /* SafeTensorsStats (safetensors.h:50-61) */
    uint64_t total, accepted, rejected;
    uint64_t duplicate_rejected, dtype_rejected, f32_allowed_accepted;
    uint64_t shape_rejected, bounds_rejected, byte_mismatch_rejected, alignment_rejected;
    int32_t shards;
    int32_t reserved;
} hfmoe_safetensors_stats;

typedef struct hfmoe_tensor_info {  /* TensorInfo / TensorLocation (weight_index.h:14-26) */
    char dtype[8];
    int32_t ndim;
    int32_t reserved;
    int64_t shape[8];
    uint64_t nbytes;
    uint64_t file_offset;  /* absolute byte offset of the data in its shard */
} hfmoe_tensor_info;

/* path: a directory of *.safetensors shards (with model.safetensors.index.json
 * when present: its weight_map picks each tensor's shard), or one shard file.
 * Parsing needs no device.  Fails on an unreadable shard, a header length that
 * is not a multiple of 8 or a header that is not a JSON object. */
int hfmoe_checkpoint_open(const char* path, hfmoe_checkpoint** out);
int hfmoe_checkpoint_stats(const hfmoe_checkpoint* ck, hfmoe_safetensors_stats* out);
int hfmoe_checkpoint_tensor(const hfmoe_checkpoint* ck, const char* name, hfmoe_tensor_info* out);
/* Copies model.layers.<layer>.mlp.{gate.weight, gate.e_score_correction_bias,
 * shared_experts.*, experts.<e>.{gate,up,down}_proj.weight} and
 * post_attention_layernorm.weight (shapes checked against hfmoe_configure) to
 * HBM -- routed experts to HBM or pinned host RAM per experts_location, each
 * expert as [gate | up | down] (scheduler.cpp:437-471) -- and registers the
 * layer.  The checkpoint owns these copies. */
int hfmoe_checkpoint_load_moe_layer(hfmoe_checkpoint* ck, int layer, int experts_location);
/* model.layers.<layer>.mlp.{gate,up,down}_proj.weight (+ post_attention_layernorm)
 * of a dense layer to HBM, intermediate size from the tensors; registers it
 * with hfmoe_register_dense_layer. */
int hfmoe_checkpoint_load_dense_layer(hfmoe_checkpoint* ck, int layer);
/* lm_head.weight (+ model.norm.weight) to HBM; registers the LM head. */
int hfmoe_checkpoint_load_lm_head(hfmoe_checkpoint* ck);
/* Unregisters the layers (and LM head) loaded from ck, frees their copies and the index. */
void hfmoe_checkpoint_close(hfmoe_checkpoint* ck);

/* ---- telemetry (InferenceStats gpuActiveNs / pcieBytes,
 *      src/engine/inference_stats.h:86-93) ---- */
typedef struct hfmoe_kernel_stat {
    char name[32];
    int64_t launches;
    double total_ms;   /* sum of hipEvent-measured durations on the launch stream */
} hfmoe_kernel_stat;

int hfmoe_profile_enable(int on);                 /* per-kernel hipEvent timing */
int hfmoe_profile_read(hfmoe_kernel_stat* out, int max_entries, int* n_entries);
int hfmoe_profile_reset(void);
int hfmoe_stats(uint64_t* pcie_bytes, uint64_t* gpu_active_ns);

#ifdef __cplusplus
}
#endif
#endif
