/*
 * libirodori_hip — MI355X (gfx950) implementation of the Irodori-TTS rectified-flow DiT
 * step, behind a plain C ABI (no HIP or torch types in any signature).
 *
 * What it replaces in the reference (Sanzentyo/Irodori-TTS-burn):
 *   - the per-step DiT forward InferenceOptimizedModel::forward_with_cond_cached
 *     (src/model/optimized.rs:102-113 -> src/model/dit/model.rs:249-262, 354-393);
 *   - the Joint-CFG Euler loop of sample_euler_rf_cfg
 *     (src/rf/euler_sampler.rs:132-718, Joint branch :435-469, update :714);
 *   - the per-layer context KV cache CondKvCache (src/model/attention.rs:24-45);
 *   - the operator entry points of src/kernels (rms_norm_wgsl rms_norm.rs:70-142,
 *     fused_adaln_wgsl fused_adaln.rs:92-205, native_fa_sdpa_wgsl
 *     fused_sdpa_native.rs:220-302, native_fa_sdpa_f16_in fused_sdpa_native_f16.rs:181).
 *
 * Conventions
 *   - Every call returns an int status (IRODORI_OK or an IRODORI_ERR_* code) and never
 *     aborts; irodori_last_error() returns the calling thread's last message.  This
 *     replaces the reference's assert!-panics and maps onto IrodoriError
 *     (src/error.rs:4-60).
 *   - Host weight pointers are float32 in Burn "row" layout [d_in, d_out], y = x @ W + b
 *     (src/weights/record_builders.rs:37-66).  The library copies and re-lays them out
 *     in device memory; the caller keeps ownership of every host buffer.
 *   - A context owns its HIP streams, its device buffers and its captured graphs.  It is
 *     single-threaded (not re-entrant); use one context per thread.
 *   - Sampler rows are role-major: role r of utterance u is batch row r * U + u.  Role 0
 *     is the conditioned bundle; with cfg_mode Joint, role 1 is the unconditioned bundle
 *     (EncodedCondition::zeros_like, condition.rs:144-154); with Independent or
 *     Alternating, role 1 + k is the bundle with the k-th active CFG signal dropped
 *     (make_single_uncond, euler_sampler.rs:41-85), the signals ordered text, speaker,
 *     caption and active when their scale is > 0 (speaker: has_speaker; caption:
 *     has_caption).  A dropped signal has zero K/V and all of its keys masked.
 */
#ifndef IRODORI_HIP_H
#define IRODORI_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (IrodoriError variants, src/error.rs:4-60) ---------------------- */
#define IRODORI_OK 0
#define IRODORI_ERR_INVALID_ARG 1 /* null pointer, out-of-range index */
#define IRODORI_ERR_SHAPE 2       /* dimension mismatch / unsupported shape */
#define IRODORI_ERR_DTYPE 3       /* unsupported dtype */
#define IRODORI_ERR_HIP 4         /* HIP runtime error */
#define IRODORI_ERR_OOM 5         /* device allocation failed (or would pass the limit that the
                                     environment variable IRODORI_DEVICE_ALLOC_LIMIT, a byte
                                     count, sets on each context's, encoder's and codec's
                                     persistent device buffers: a way to exercise this path) */
#define IRODORI_ERR_NOT_LOADED 6  /* weights / context KV missing */
#define IRODORI_ERR_CONFIG 7      /* invalid sampler / model configuration */

#define IRODORI_DTYPE_F32 0
#define IRODORI_DTYPE_BF16 1
/* bf16 activations and attention; the block GEMMs (QKV+gate, W_o, W1|W3, W2) on e4m3fn
 * operands: weights with one f32 scale per output channel, GEMM inputs with one
 * power-of-two scale per 32 values along k (the gfx950 scaled fp8 MFMA).  No counterpart in
 * the reference (fp8 weights for batched throughput); needs model_dim, mlp_hidden % 128 == 0. */
#define IRODORI_DTYPE_FP8 2
/* IEEE half storage with f32 arithmetic: the Q/K/V dtype of native_fa_sdpa_f16_in
 * (fused_sdpa_native_f16.rs:181-200); accepted by irodori_op_sdpa only. */
#define IRODORI_DTYPE_F16 3

#define IRODORI_CFG_INDEPENDENT 0 /* CfgGuidanceMode (src/config/sampling.rs:100-108) */
#define IRODORI_CFG_JOINT 1
#define IRODORI_CFG_ALTERNATING 2

#define IRODORI_METHOD_EULER 0 /* SamplerMethod (src/config/sampling.rs:8-20) */
#define IRODORI_METHOD_HEUN 1
#define IRODORI_METHOD_PLMS4 2

typedef struct irodori_ctx irodori_ctx;

/* Model dimensions: the ModelConfig fields the DiT forward reads
 * (src/config/model.rs:8-44), plus device sizing. */
typedef struct irodori_dit_config {
    int32_t latent_dim;         /* patched latent dim P (latent_dim * latent_patch_size), <= 256 */
    int32_t model_dim;          /* D, a multiple of 64, <= 4096 */
    int32_t num_layers;         /* L */
    int32_t num_heads;          /* H (head_dim = D / H) */
    int32_t head_dim;           /* Dh: 64, or 128 for bf16 / f32 (fp8 compute needs 64) */
    int32_t mlp_hidden;         /* F = floor(D * mlp_ratio) (diffusion.rs:32), multiple of 16 */
    int32_t adaln_rank;         /* r (norm.rs:101-104) */
    int32_t timestep_embed_dim; /* t_dim */
    float norm_eps;             /* norm_eps (config/model.rs:78) */
    float rope_theta;           /* 10000 (dit/model.rs:216) */
    int32_t compute_dtype;      /* IRODORI_DTYPE_BF16 (MFMA bf16), _F32 or _FP8 */
    int32_t max_rows;           /* max batch rows in one forward (2 per utterance), <= 65535 */
    int32_t max_seq;            /* max latent frames S */
    int32_t max_ctx;            /* max context keys T = text + speaker */
} irodori_dit_config;

/* One DiffusionBlock (src/model/diffusion.rs:21-28) in the fused inference layout
 * (attention.rs:514-523, feed_forward.rs:96-103).  adaLN index [0] = attention_adaln,
 * [1] = mlp_adaln; chunk index [0] = shift, [1] = scale, [2] = gate (norm.rs:141-157). */
typedef struct irodori_block_weights {
    const float* w_qkv;          /* [D, 3*H*Dh] = [Wq | Wk | Wv] */
    const float* w_gate;         /* [D, D] attention output gate */
    const float* w_o;            /* [H*Dh, D] */
    const float* q_norm;         /* [H, Dh] */
    const float* k_norm;         /* [H, Dh] */
    const float* w13;            /* [D, 2F] = [W1 | W3] */
    const float* w2;             /* [F, D] */
    const float* ada_down[2][3]; /* [D, r], no bias */
    const float* ada_up[2][3];   /* [r, D] */
    const float* ada_up_b[2][3]; /* [D] */
} irodori_block_weights;

/* Per-forward weights outside the blocks (src/model/dit/model.rs:104-125). */
typedef struct irodori_io_weights {
    const float* cond_w0;    /* cond_module.0 [t_dim, D] */
    const float* cond_w1;    /* cond_module.2 [D, D] */
    const float* cond_w2;    /* cond_module.4 [D, 3D] */
    const float* in_w;       /* in_proj [P, D] */
    const float* in_b;       /* [D] */
    const float* out_norm_w; /* out_norm [D] */
    const float* out_w;      /* out_proj [D, P] */
    const float* out_b;      /* [P] */
} irodori_io_weights;

/* SamplerParams + GuidanceConfig + TemporalRescaleConfig + SpeakerKvConfig
 * (src/rf/params.rs:9-92) and the request facts that select the active CFG signals
 * (euler_sampler.rs:163-200). */
typedef struct irodori_sampler_params {
    int32_t num_steps;
    int32_t method;   /* IRODORI_METHOD_* */
    int32_t cfg_mode; /* IRODORI_CFG_* */
    float scale_text;
    float scale_caption;
    float scale_speaker;
    float min_t;
    float max_t;
    int32_t has_truncation;
    float truncation_factor;
    int32_t has_speaker;  /* the model uses speaker conditioning and the condition holds a speaker state */
    int32_t has_caption;  /* the condition holds a caption with at least one valid token */
    int32_t has_temporal_rescale; /* temporal_score_rescale (math.rs:38-53) with k, sigma */
    float rescale_k;
    float rescale_sigma;
    int32_t has_speaker_kv;       /* force-speaker KV scaling (kv_scaling.rs:10-60) */
    float speaker_kv_scale;
    int32_t speaker_kv_max_layers; /* < 0: every layer */
    int32_t speaker_kv_has_min_t;  /* revert the scaling once t drops below speaker_kv_min_t */
    float speaker_kv_min_t;
    int32_t ctx_aux_start;         /* first aux (speaker) key of the context sequence (= text keys) */
} irodori_sampler_params;

/* ---- errors ----------------------------------------------------------------------- */
const char* irodori_last_error(void);
const char* irodori_version(void);

/* SamplerParams::validate (params.rs:99-183) plus the Joint equal-scale rule
 * (euler_sampler.rs:209-228).  Pure host logic: no device needed. */
int irodori_sampler_params_validate(const irodori_sampler_params* params);

/* ---- context ---------------------------------------------------------------------- */
/* Creates a context on HIP device `device`; allocates every device buffer up front for
 * cfg->max_rows / max_seq / max_ctx.  Replaces InferenceBuilder::build
 * (src/inference.rs:83-196) for the HIP backend.  bf16 / fp8 contexts take at most 16384
 * keys per attention row: ceil(max_seq / 64) + ceil(max_ctx / 64) <= 256, else
 * IRODORI_ERR_SHAPE here (never at a later launch). */
int irodori_ctx_create(int device, const irodori_dit_config* cfg, irodori_ctx** out);
int irodori_ctx_destroy(irodori_ctx* ctx);
/* Bytes of device memory the context holds. */
int irodori_ctx_device_bytes(const irodori_ctx* ctx, uint64_t* bytes);

/* Weight ingest (load_model -> InferenceOptimizedModel::from, inference.rs:107-116,
 * :187-195): host f32 in Burn layout -> device compute dtype, fused layouts. */
int irodori_load_io_weights(irodori_ctx* ctx, const irodori_io_weights* w);
int irodori_load_block_weights(irodori_ctx* ctx, int layer, const irodori_block_weights* w);

/* Context KV for one layer and one batch row: the CondKvCache contents
 * (attention.rs:24-45; built by build_kv_cache :431-501).  k, v: [t_ctx, H, Dh] f32,
 * k already k-normed and not rotated; mask: [t_ctx] (nonzero = attend).  Every row and
 * layer must use the same t_ctx (<= max_ctx); irodori_clear_ctx_kv resets it. */
int irodori_set_ctx_kv(irodori_ctx* ctx, int layer, int row, int t_ctx, const float* k,
                       const float* v, const uint8_t* mask);
int irodori_clear_ctx_kv(irodori_ctx* ctx);

/* Context projections of one layer, JointAttention wk_text / wv_text and wk_speaker /
 * wv_speaker (or the caption pair) (attention.rs:142-147, :183-207): Burn [d_in, H*Dh],
 * no bias.  aux pointers may be NULL when aux_dim is 0.  Every layer must use the same
 * text_dim / aux_dim. */
typedef struct irodori_ctx_proj_weights {
    const float* wk_text; /* [text_dim, H*Dh] */
    const float* wv_text;
    const float* wk_aux;  /* [aux_dim, H*Dh] */
    const float* wv_aux;
} irodori_ctx_proj_weights;
int irodori_load_ctx_proj_weights(irodori_ctx* ctx, int layer, int text_dim, int aux_dim,
                                  const irodori_ctx_proj_weights* w);

/* build_kv_cache (attention.rs:431-501) on the device for every layer and one batch row:
 * K = k_norm(state @ Wk) (not rotated), V = state @ Wv for the text state [t_text, text_dim]
 * and the aux state [t_aux, aux_dim] (nullable when t_aux = 0), concatenated [text | aux]
 * with ctx_mask = [text_mask | aux_mask] (nonzero = attend).  Replaces irodori_set_ctx_kv
 * for that row (same t_ctx rule: t_text + t_aux).  An unconditioned bundle is built from
 * zero states with all-false masks (condition.rs:144-154).  Host pointers; synchronous. */
int irodori_build_ctx_kv(irodori_ctx* ctx, int row, int t_text, const float* text_state,
                         const uint8_t* text_mask, int t_aux, const float* aux_state,
                         const uint8_t* aux_mask);

/* Inspection (no counterpart in the reference, which keeps CondKvCache as tensors): copy
 * the cached context of one layer and batch row back to the host as k, v [t_ctx, H, Dh]
 * (k normed, not rotated) and mask [t_ctx], in the compute dtype's values.  Synchronous. */
int irodori_read_ctx_kv(irodori_ctx* ctx, int layer, int row, float* k, float* v, uint8_t* mask);

/* One DiT forward, forward_with_cond_cached (optimized.rs:102-113): x_t [B,S,P],
 * t [B] -> v [B,S,P].  debug (nullable): [L+1,B,S,D] after in_proj and after each block
 * (BlockDebugOutputs, dit/model.rs:92-102).  Host pointers; synchronous. */
int irodori_forward(irodori_ctx* ctx, int batch, int seq, const float* x_t, const float* t,
                    float* v_out, float* debug);

/* forward_with_cond_cached with a latent mask (optimized.rs:102-113 latent_mask;
 * build_joint_mask, attention.rs:730-750): latent_mask [B,S] (nonzero = the latent key
 * attends; NULL = all attend) masks latent keys in every block's joint attention.  Query
 * rows are computed for every frame; a row with no valid key gets a zero attention output. */
int irodori_forward_masked(irodori_ctx* ctx, int batch, int seq, const float* x_t, const float* t,
                           const uint8_t* latent_mask, float* v_out, float* debug);

/* One DiffusionBlock::forward_fused (diffusion.rs:62-105) on host data:
 * x [B,S,D] updated in place; cond [B,3D] is the cond_module output. */
int irodori_block_forward(irodori_ctx* ctx, int layer, int batch, int seq, float* x,
                          const float* cond);

/* RF sampling (sample_euler_rf_cfg, euler_sampler.rs:132-718): U utterances, x0 [U,S,P]
 * -> x_out [U,S,P], every cfg_mode (rows role-major, see the conventions above) and method
 * (Euler; Heun at 2 forwards per step; PLMS-4), temporal score rescaling and speaker-KV
 * scaling.  A step's forward runs only the roles it needs (the conditioned role alone
 * outside the CFG window; Alternating the conditioned role and the role dropped at that
 * step), each role as its own kernel chain of a captured hipGraph.  Host pointers.
 * Truncation (params.rs:146-155) is applied to x0 when set. */
int irodori_sample(irodori_ctx* ctx, const irodori_sampler_params* params, int utterances,
                   int seq, const float* x0, float* x_out);
/* Sampling of a padded variable-length batch: utterance u attends to its first
 * lengths[u] latent frames (in every role), so frames below lengths[u] match an unpadded
 * run of that utterance (padded batches of utterances; the reference sampler always
 * passes latent_mask = None, euler_sampler.rs:410-523).  lengths: host int32 [U]. */
int irodori_sample_masked(irodori_ctx* ctx, const irodori_sampler_params* params, int utterances,
                          int seq, const int32_t* lengths, const float* x0, float* x_out);
/* Same with x0 / x_out already in device memory (HBM-resident timing). */
int irodori_sample_device(irodori_ctx* ctx, const irodori_sampler_params* params,
                          int utterances, int seq, const float* d_x0, float* d_x_out);
/* irodori_sample_masked with x0 / x_out in device memory; lengths stays a host array. */
int irodori_sample_device_masked(irodori_ctx* ctx, const irodori_sampler_params* params,
                                 int utterances, int seq, const int32_t* lengths,
                                 const float* d_x0, float* d_x_out);

/* ---- isolated block operators on a loaded context --------------------------------------
 * The block's hot kernels alone, on the context's weights of `layer` (loaded in the kernels'
 * layouts), with device pointers, enqueued on `stream` (NULL: the context's stream) without
 * waiting.  They use the context's work buffers: calls that overlap with each other or with
 * a forward / sampling call on the same context race. */

/* attention_after_qkv (attention.rs:328-425) of one block: the latent projections q, k, v
 * [batch, seq, H, 64] f32 (before the head norms), head-normed with the layer's q_norm /
 * k_norm, half-RoPE'd at latent positions 0..seq-1 (rope.rs:119-135), joined with the
 * layer's cached context keys / values / mask of rows 0..batch-1 (irodori_set_ctx_kv or
 * irodori_build_ctx_kv; the keys are normed, not rotated), SDPA (attention.rs:619-664; a
 * row with no valid key gives 0), then sigmoid(gate) times the output (gate: logits
 * [batch, seq, H*64] f32, nullable = 1, attention.rs:423).  out [batch, seq, H*64] f32.
 * Runs the model's attention kernel on the layouts its QKV+gate epilogue writes.  bf16 or
 * f32 contexts. */
int irodori_op_joint_attention(irodori_ctx* ctx, int layer, int batch, int seq, const float* q,
                               const float* k, const float* v, const float* gate, float* out,
                               void* stream);

/* The MLP half of DiffusionBlock::forward_fused (diffusion.rs:101-104) of one block:
 * x += gate * SwiGlu(x / rms(x) * (1 + scale) + shift) (norm.rs:160-169,
 * feed_forward.rs:76-85), with the caller's modulation vectors shift / scale / gate
 * [batch, D] f32 (gate as applied, after tanh) and the context's norm_eps; x [batch, seq, D]
 * f32, updated in place.  bf16 contexts with the fused adaLN run each row as a sampler
 * chain does (the norm folded into the W1|W3 GEMM); otherwise the adaLN kernel, W1|W3 and W2
 * over all rows.  Overwrites the context's modulation table rows 0..batch-1 of (layer,
 * mlp), which the next forward or sampling call rebuilds. */
int irodori_op_swiglu_mlp(irodori_ctx* ctx, int layer, int batch, int seq, float* x,
                          const float* shift, const float* scale, const float* gate, void* stream);

/* Average device time of each kernel of one DiT block over `batch` rows of `seq` frames,
 * launched as one sampler role chain launches them (every row on the same timestep's
 * modulation vector; batch = 1 is one CFG row of a Joint-CFG step), measured with HIP
 * events on the context's stream over `iters` back-to-back launches per kernel, launch i
 * using layer i % num_layers (weights and context K/V cycle through the layers as in an RF
 * step) -- the reference's NVTX per-call timings (docs/benchmarks/rtx-a6000.md:131-138) as
 * a measurement entry point.  norm_mod_us times the unfused adaLN kernel, which the
 * sampler's bf16 chains fold into their GEMMs.  bf16 contexts (an fp8 context times its
 * fp8 GEMMs); weights and context KV must be loaded.  Microseconds. */
typedef struct irodori_kernel_times {
    float norm_mod_us;   /* unfused RMSNorm + adaLN modulation kernel (x f32 -> h bf16), each
                            launch on its own buffers from a >= 640 MB pool (cold HBM) */
    float qkvg_gemm_us;  /* QKV + gate projection with head norm / RoPE epilogue */
    float attention_us;  /* joint flash attention + sigmoid gate */
    float wo_gemm_us;    /* output projection + gated residual */
    float w13_gemm_us;   /* SwiGLU up-projection with silu(a)*b epilogue */
    float w2_gemm_us;    /* SwiGLU down-projection + gated residual */
    float final_us;      /* out_norm + out_proj + CFG combine + Euler update */
} irodori_kernel_times;
int irodori_profile_layer(irodori_ctx* ctx, int batch, int seq, int iters,
                          irodori_kernel_times* out);

/* Replaces the reference's NVTX ranges (src/profiling.rs:29-92, compiled in by its `profile`
 * feature; used at src/model/dit/model.rs:238-392, src/model/diffusion.rs:88-158,
 * src/rf/euler_sampler.rs:409-580): the library marks the same spans with roctx ranges of the
 * same names (dit_forward_with_cond_fused, timestep_embed, cond_module, in_proj, dit_block_<i>,
 * adaln_attn, joint_attention_fused, adaln_mlp, swiglu_mlp_fused, out_proj,
 * forward_batched_cfg, forward_cond, forward_uncond, heun_corrector) for rocprofv3
 * --marker-trace when the process runs with IRODORI_ROCTX=1 (read once, at the first range;
 * the roctx library is then loaded at run time).  Returns 1 when ranges are on, else 0. */
int irodori_roctx_enabled(void);

/* ---- condition encoders ---------------------------------------------------------------
 * TextEncoder (text / caption, text_encoder.rs:64-148) and ReferenceLatentEncoder (speaker,
 * speaker_encoder.rs:85-162) with their conditioner norm (text_norm, dit/model.rs:189-190;
 * aux_conditioner.rs:60-85) and, for the speaker, the masked-mean token
 * (aux_conditioner.rs:150-185): EncodedCondition's text_state / aux state on the device.
 * The reference runs these once per request on the CPU backend; here they run on the GPU
 * (compute_dtype BF16: bf16 GEMM / attention operands, f32 residual; F32: f32 throughout). */
typedef struct irodori_encoder irodori_encoder;

typedef struct irodori_encoder_config {
    int32_t dim;           /* text_dim / speaker_dim / caption_dim */
    int32_t num_layers;
    int32_t num_heads;     /* head_dim = dim / num_heads: 64 or 128 */
    int32_t mlp_hidden;    /* floor(dim * mlp_ratio) (text_encoder.rs:36), multiple of 16 */
    int32_t vocab_size;    /* > 0: token ids in (TextEncoder), embedding [vocab, dim] */
    int32_t in_dim;        /* > 0: latent frames in (ReferenceLatentEncoder), in_proj [in_dim, dim] */
    int32_t mean_token;    /* 1: prepend the speaker conditioner's masked-mean token */
    float norm_eps;
    int32_t compute_dtype; /* IRODORI_DTYPE_BF16 or IRODORI_DTYPE_F32 */
    int32_t max_rows;      /* max batch rows */
    int32_t max_seq;       /* max tokens / frames per row */
} irodori_encoder_config;

/* Front end and conditioner norm, Burn layouts, host f32; unused pointers may be NULL. */
typedef struct irodori_encoder_io_weights {
    const float* embedding; /* [vocab, dim] text_embedding.weight */
    const float* in_w;      /* [in_dim, dim] in_proj.weight */
    const float* in_b;      /* [dim] in_proj.bias */
    const float* out_norm;  /* [dim] text_norm / speaker or caption conditioner norm weight */
} irodori_encoder_io_weights;

/* One TextBlock (text_encoder.rs:17-60): attention_norm, SelfAttention (wq, wk, wv, wo,
 * gate, q_norm, k_norm; attention.rs:52-127), mlp_norm, SwiGlu (w13 = [W1 | W3], w2). */
typedef struct irodori_encoder_block_weights {
    const float* attn_norm; /* [dim] */
    const float* wq;        /* [dim, dim] */
    const float* wk;
    const float* wv;
    const float* wo;        /* [dim, dim] */
    const float* w_gate;    /* [dim, dim] */
    const float* q_norm;    /* [heads, head_dim] */
    const float* k_norm;
    const float* mlp_norm;  /* [dim] */
    const float* w13;       /* [dim, 2 * mlp_hidden] */
    const float* w2;        /* [mlp_hidden, dim] */
} irodori_encoder_block_weights;

int irodori_encoder_create(int device, const irodori_encoder_config* cfg, irodori_encoder** out);
int irodori_encoder_destroy(irodori_encoder* enc);
int irodori_encoder_load_io_weights(irodori_encoder* enc, const irodori_encoder_io_weights* w);
int irodori_encoder_load_block_weights(irodori_encoder* enc, int layer,
                                       const irodori_encoder_block_weights* w);
/* Encode `batch` rows of `seq` tokens (ids [batch, seq], vocab_size > 0) or latent frames
 * (latent [batch, seq, in_dim], in_dim > 0); mask [batch, seq] (nonzero = valid).
 * state_out [batch, seq + mean_token, dim] f32; mask_out (nullable) [batch, seq +
 * mean_token].  Host pointers; synchronous. */
int irodori_encoder_forward(irodori_encoder* enc, int batch, int seq, const int32_t* ids,
                            const float* latent, const uint8_t* mask, float* state_out,
                            uint8_t* mask_out);

/* ---- DACVAE decoder -------------------------------------------------------------------
 * DacVaeCodec::decode (codec/model.rs:60-65): latent [B, T, latent_dim] -> waveform
 * [B, 1, T * hop], hop = prod(rates): quantizer.out_proj (bottleneck.rs:21-23), the decoder
 * stem, DecoderBlocks (Snake, ConvTranspose1d(kernel 2r, stride r, padding ceil(r/2),
 * output padding r % 2), ResidualUnits of dilation 1, 3, 9) and the watermark head (Snake,
 * Conv1d(-> 1, kernel 7), tanh) of codec/decoder.rs, as built by codec/weights.rs:225-292
 * (load_codec).  The reference decodes on its CPU/WGPU backend; here the convolutions run
 * on the matrix cores (BF16: bf16 operands, f32 accumulation and residual stream; F32: f32
 * throughout). */
#define IRODORI_CODEC_MAX_BLOCKS 8

typedef struct irodori_codec irodori_codec;

typedef struct irodori_codec_config {
    int32_t latent_dim;    /* 32: codebook_dim (bottleneck.rs); <= 1024 */
    int32_t proj_dim;      /* 1024: quantizer.out_proj output channels, multiple of 8 */
    int32_t decoder_dim;   /* 1536: stem output; block i maps dim >> i to dim >> (i + 1) */
    int32_t num_blocks;    /* 4, at most IRODORI_CODEC_MAX_BLOCKS */
    int32_t rates[IRODORI_CODEC_MAX_BLOCKS]; /* 12, 10, 8, 2; each in [2, 64] */
    int32_t compute_dtype; /* IRODORI_DTYPE_BF16 or IRODORI_DTYPE_F32 */
    int32_t max_frames;    /* max latent frames per row */
} irodori_codec_config;

/* One DecoderBlock (decoder.model.{1..}: block.0 Snake, block.1 ConvTranspose1d, block.4 /
 * .5 / .8 ResidualUnits with block.0 Snake, block.1 Conv1d k 7, block.2 Snake, block.3
 * Conv1d k 1).  Burn layouts, host f32; biases may be NULL. */
typedef struct irodori_codec_block_weights {
    const float* alpha;          /* [in] */
    const float* convt_w;        /* [in, out, 2 rate] */
    const float* convt_b;        /* [out] */
    const float* res_alpha0[3];  /* [out] */
    const float* res_conv_w[3];  /* [out, out, 7], dilation 1, 3, 9 */
    const float* res_conv_b[3];  /* [out] */
    const float* res_alpha1[3];  /* [out] */
    const float* res_pw_w[3];    /* [out, out, 1] */
    const float* res_pw_b[3];    /* [out] */
} irodori_codec_block_weights;

typedef struct irodori_codec_weights {
    const float* out_proj_w;  /* [proj_dim, latent_dim, 1] quantizer.out_proj */
    const float* out_proj_b;  /* [proj_dim] */
    const float* stem_w;      /* [decoder_dim, proj_dim, 7] decoder.model.0 */
    const float* stem_b;      /* [decoder_dim] */
    const irodori_codec_block_weights* blocks; /* [num_blocks] */
    const float* head_alpha;  /* [decoder_dim >> num_blocks] wm_model.encoder_block.pre.0 */
    const float* head_w;      /* [1, decoder_dim >> num_blocks, 7] pre.1 */
    const float* head_b;      /* [1] */
} irodori_codec_weights;

int irodori_codec_create(int device, const irodori_codec_config* cfg, irodori_codec** out);
int irodori_codec_destroy(irodori_codec* codec);
int irodori_codec_load_weights(irodori_codec* codec, const irodori_codec_weights* w);
/* hop_length (codec/model.rs): waveform samples per latent frame, prod(rates). */
int irodori_codec_hop_length(const irodori_codec* codec);
/* latent [batch, frames, latent_dim] -> wav [batch, frames * hop] f32; host pointers,
 * synchronous. */
int irodori_codec_decode(irodori_codec* codec, int batch, int frames, const float* latent,
                         float* wav);
/* The same on device pointers, enqueued on `stream` (NULL: the codec's own stream) without
 * waiting.  Rows run one after another on the codec's work buffers, so calls that overlap
 * on one codec (on different streams, or from different threads) race. */
int irodori_codec_decode_device(irodori_codec* codec, int batch, int frames,
                                const float* latent, float* wav, void* stream);

/* ---- operator entry points (device pointers; stream may be NULL) ------------------- */
/* rms_norm_wgsl (rms_norm.rs:70-142): y = x / sqrt(mean(x^2)+eps) * w, x [rows, dim]. */
int irodori_op_rms_norm(const float* x, const float* w, int rows, int dim, float eps,
                        float* y, void* stream);
/* fused_adaln_wgsl (fused_adaln.rs:92-205): y = x/rms * (1 + scale[b]) + shift[b],
 * x [batch*seq, dim], scale/shift [batch, dim]. */
int irodori_op_fused_adaln(const float* x, const float* scale, const float* shift, int batch,
                           int seq, int dim, float eps, float* y, void* stream);
/* native_fa_sdpa_wgsl / native_fa_sdpa_f16_in (fused_sdpa_native.rs:220-302,
 * fused_sdpa_native_f16.rs:181-200), and fused_sdpa_wgsl / tiled_fa_sdpa_wgsl
 * (fused_sdpa.rs:107, fused_sdpa_tiled.rs:202), which take the same tensors and differ only
 * in their WGSL tiling config: out = softmax(q k^T * scale + mask) v.
 * q [B,H,Sq,Dh], k/v [B,H,Skv,Dh] in `dtype` (F32, BF16 or F16: native_fa_sdpa_f16_in's
 * f16 storage, f32 accumulation), mask [B,Skv] f32 with 1.0 = attend (values < 0.5 mask
 * the key; may be NULL), out [B,H,Sq,Dh] f32.  Dh in {64, 128}.  A fully masked query row
 * yields 0.  Enqueued on `stream` without waiting.  With Dh = 64, a 16-bit dtype and
 * seq_kv <= 16384 the call stages Q (pre-scaled), V^T and the key bits in a device buffer it
 * allocates and frees in stream order on `stream` (hipMallocAsync / hipFreeAsync), and runs
 * the model's joint attention kernel on them; other shapes need no staging and run the
 * generic flash kernel, whose softmax is f32 throughout.  Precision of the staged path: the
 * scores and the softmax state are f32, but q * scale * log2(e) and the probabilities P
 * (the P V MFMA operand) are rounded to the operand dtype, as the model's bf16 attention
 * does; the reference's native FA kernels keep both in f32.  Measured against a float64
 * SDPA of the same rounded inputs at config 2's shape: 2.4e-3 relative L2 in bf16 and
 * 3.0e-4 in f16 (bars 1e-2 and 2e-3; max abs 1.5e-3 and 2.0e-4). */
int irodori_op_sdpa(int dtype, const void* q, const void* k, const void* v, const float* mask,
                    int batch, int heads, int seq_q, int seq_kv, int head_dim, float scale,
                    float* out, void* stream);
/* No counterpart in the reference: irodori_op_sdpa for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).  Same
 * arguments, kernels and results; the staging of the 16-bit head_dim-64 path lives in one
 * fixed device buffer of IRODORI_SDPA_SCRATCH_BYTES per GPU, held until the process ends,
 * instead of a per-call allocation.  A shape whose staging (Q + V^T in the operand dtype +
 * the key bits, each rounded up to 256 bytes) exceeds it returns IRODORI_ERR_SHAPE.  Every
 * call on a GPU shares that buffer: calls that overlap on one GPU (other streams or
 * threads) race.  `stream` must belong to the current device (else IRODORI_ERR_INVALID_ARG).
 * The first call on a device looks up the buffer's address and must not be made under graph
 * capture (IRODORI_ERR_INVALID_ARG): capturing callers make one call outside the capture
 * first; later calls may be captured and replayed. */
#define IRODORI_SDPA_SCRATCH_BYTES (16u << 20)
int irodori_op_sdpa_noalloc(int dtype, const void* q, const void* k, const void* v, const float* mask,
                            int batch, int heads, int seq_q, int seq_kv, int head_dim, float scale,
                            float* out, void* stream);
/* The fp8 GEMM-operand form of the IRODORI_DTYPE_FP8 mode (no counterpart in the
 * reference): x [rows, dim] f32 (dim % 32 == 0) -> e4m3 codes q [rows, dim] and E8M0 scale
 * bytes s [rows, dim/32]; per 32-wide block, 2^e with e the smallest integer such that
 * max |x| <= 448 * 2^e, codes = round-to-nearest-even e4m3(x * 2^-e). */
int irodori_op_mx_quantize(const float* x, int rows, int dim, uint8_t* q, uint8_t* s, void* stream);
/* The fp8 block GEMM of that mode: c[m, n] = w_scale[n] * sum_k a[m, k] 2^(a_scale[m, k/32] - 127)
 * * w[n, k], with a [M, K] and w [N, K] e4m3 codes (K-contiguous, K % 128 == 0, N % 64 == 0),
 * a_scale [M, K/32] E8M0 bytes, w_scale [N] f32; c [M, N] f32. */
int irodori_op_gemm_fp8(const uint8_t* a, const uint8_t* a_scale, const uint8_t* w, const float* w_scale,
                        int M, int N, int K, float* c, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* IRODORI_HIP_H */
