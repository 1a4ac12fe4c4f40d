/*
 * CPU oracle for the Irodori-TTS RF-step DiT forward — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's Burn NdArray f32 semantics for the
 * hot path (one DiT forward and the Joint-CFG Euler sampler).  It is used only by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py, as the
 * checker and as the timed CPU baseline.  The product (libirodori_hip.so) never
 * links, loads or calls it.
 *
 * Every function is compiled twice from oracle_body.h: once with float arithmetic
 * (orc_f32_*, the NdArray<f32> analogue) and once with double arithmetic
 * (orc_f64_*, the reference of record).  Inputs and outputs are always float, and so are
 * the buffers between operators: the f64 variant rounds to f32 only at operator
 * boundaries (relative ~1e-7), far below every tolerance it is used for.
 *
 * Layouts follow the reference at the Burn boundary: every Linear weight is
 * [d_in, d_out] row-major with y = x @ W + b (src/weights/record_builders.rs:37-66).
 */
#ifndef IRODORI_ORACLE_H
#define IRODORI_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_cfg {
    int32_t latent_dim;   /* patched latent dim P */
    int32_t model_dim;    /* D */
    int32_t num_layers;   /* L */
    int32_t num_heads;    /* H */
    int32_t head_dim;     /* Dh */
    int32_t mlp_hidden;   /* F */
    int32_t adaln_rank;   /* r */
    int32_t t_dim;        /* timestep embedding dim */
    float norm_eps;
    float rope_theta;
    int32_t gemm_fp8;     /* 1: the block GEMMs take fp8 operands (orc_mx_quantize_rows /
                             orc_quant_weight_cols), the HIP path's fp8 compute mode */
    int32_t fused_adaln;  /* 1: every row of a block shares one modulation vector and the
                             adaLN is folded into the GEMMs that read h, as the HIP path's
                             bf16 sampler chains compute it: h W = r (x (1 + scale)) W +
                             shift W with r = rsqrt(mean x^2 + eps) per row (with gemm_fp8
                             the GEMM inputs x (1 + scale) and the shift row would each be
                             quantized; the HIP fp8 mode keeps the unfolded adaLN) */
} orc_cfg;

/* One DiffusionBlock (src/model/diffusion.rs:21-28), fused inference layout
 * (attention.rs:514-523, feed_forward.rs:96-103).  adaln index: [0]=attention_adaln,
 * [1]=mlp_adaln; chunk index: [0]=shift, [1]=scale, [2]=gate (norm.rs:141-157). */
typedef struct orc_block {
    const float* w_qkv;   /* [D, 3*H*Dh] = [Wq | Wk | Wv] */
    const float* w_gate;  /* [D, D] */
    const float* w_o;     /* [H*Dh, D] */
    const float* q_norm;  /* [H, Dh] */
    const float* k_norm;  /* [H, Dh] */
    const float* w13;     /* [D, 2F] = [W1 | W3] */
    const float* w2;      /* [F, D] */
    const float* ada_down[2][3]; /* [D, r], no bias */
    const float* ada_up[2][3];   /* [r, D] */
    const float* ada_up_b[2][3]; /* [D] */
} orc_block;

/* Non-block weights of TextToLatentRfDiT used per forward (dit/model.rs:140-170). */
typedef struct orc_io {
    const float* cond_w0;    /* [t_dim, D], no bias */
    const float* cond_w1;    /* [D, D], no bias */
    const float* cond_w2;    /* [D, 3D], no bias */
    const float* in_w;       /* [P, D] */
    const float* in_b;       /* [D] */
    const float* out_norm_w; /* [D] */
    const float* out_w;      /* [D, P] */
    const float* out_b;      /* [P] */
} orc_io;

/* SamplerParams + GuidanceConfig + TemporalRescaleConfig + SpeakerKvConfig
 * (src/rf/params.rs:9-92) as the sampler consumes them, plus the request facts that
 * select the active CFG signals (euler_sampler.rs:163-200). */
typedef struct orc_sampler {
    int32_t num_steps;
    int32_t method;     /* 0 Euler, 1 Heun, 2 PLMS-4 (config/sampling.rs:8-20) */
    int32_t cfg_mode;   /* 0 Independent, 1 Joint, 2 Alternating (config/sampling.rs:100-108) */
    float scale_text, scale_caption, scale_speaker;
    float min_t, max_t;
    int32_t has_truncation;
    float truncation_factor;
    int32_t has_speaker;  /* the model uses speaker conditioning and the condition holds a speaker state */
    int32_t has_caption;  /* the condition holds a caption with at least one valid token */
    int32_t has_temporal_rescale;
    float rescale_k, rescale_sigma;
    int32_t has_speaker_kv;
    float speaker_kv_scale;
    int32_t speaker_kv_max_layers;  /* < 0: every layer */
    int32_t speaker_kv_has_min_t;
    float speaker_kv_min_t;
    int32_t ctx_aux_start;  /* first aux (speaker) key of the context sequence */
} orc_sampler;

/* Condition encoders (text_encoder.rs:17-148, speaker_encoder.rs:85-162): a stack of
 * TextBlocks of width E = dim, H heads of Dh = E / H, SwiGLU hidden F. */
typedef struct orc_enc_cfg {
    int32_t dim;          /* E */
    int32_t num_layers;
    int32_t num_heads;    /* H */
    int32_t mlp_hidden;   /* F */
    float norm_eps;
} orc_enc_cfg;

/* One TextBlock (text_encoder.rs:17-60) with its SelfAttention (attention.rs:52-127),
 * Burn [d_in, d_out] layouts. */
typedef struct orc_enc_block {
    const float* attn_norm;  /* [E] attention_norm.weight */
    const float* wq;         /* [E, H*Dh] */
    const float* wk;
    const float* wv;
    const float* wo;         /* [H*Dh, E] */
    const float* w_gate;     /* [E, E] */
    const float* q_norm;     /* [H, Dh] */
    const float* k_norm;
    const float* mlp_norm;   /* [E] mlp_norm.weight */
    const float* w13;        /* [E, 2F] = [W1 | W3] */
    const float* w2;         /* [F, E] */
} orc_enc_block;

/* DACVAE decoder (src/codec/decoder.rs, layers.rs, bottleneck.rs; built in weights.rs:
 * 225-292): out_proj Conv1d(latent -> proj, k 1), stem Conv1d(proj -> dim, k 7), blocks i
 * (Snake, ConvTranspose1d(dim_i -> dim_i / 2, k 2 r_i, stride r_i), ResidualUnits with
 * dilations 1, 3, 9), head (Snake, Conv1d(-> 1, k 7), tanh).  Burn layouts: Conv1d weight
 * [out, in, k], ConvTranspose1d weight [in, out, k]; Snake alpha [C]. */
typedef struct orc_codec_block {
    const float* alpha;        /* [in] */
    const float* convt_w;      /* [in, out, 2 r] */
    const float* convt_b;      /* [out] */
    const float* res_alpha0[3];
    const float* res_conv_w[3];  /* [out, out, 7] */
    const float* res_conv_b[3];
    const float* res_alpha1[3];
    const float* res_pw_w[3];    /* [out, out, 1] */
    const float* res_pw_b[3];
} orc_codec_block;

typedef struct orc_codec {
    int32_t latent_dim, proj_dim, decoder_dim, num_blocks;
    int32_t rates[8];
    const float* out_proj_w;  /* [proj, latent, 1] */
    const float* out_proj_b;
    const float* stem_w;      /* [dim, proj, 7] */
    const float* stem_b;
    const orc_codec_block* blocks;
    const float* head_alpha;  /* [dim >> num_blocks] */
    const float* head_w;      /* [1, dim >> num_blocks, 7] */
    const float* head_b;      /* [1] */
} orc_codec;

/* fp8 (e4m3fn) GEMM operands (oracle.c). */
uint8_t orc_e4m3_encode(float x);
float orc_e4m3_decode(uint8_t b);
int orc_mx_scale_exp(float amax);
void orc_mx_quantize_rows(const float* x, int M, int K, uint8_t* q, uint8_t* s);
void orc_mx_dequantize_rows(const uint8_t* q, const uint8_t* s, int M, int K, float* y);
void orc_quant_weight_cols(const float* w, int K, int N, uint8_t* q, float* scale);

/* Number of OpenMP threads the oracle uses (0 = runtime default). */
void orc_set_threads(int n);
int orc_get_threads(void);

#define ORC_DECLARE(P)                                                                      \
    void P##timestep_embedding(const float* t, int B, int t_dim, float* out);              \
    void P##rope_tables(int S, int Dh, float theta, float* cos_out, float* sin_out);       \
    void P##linear(const float* x, const float* w, const float* b, int M, int K, int N,    \
                   float* y);                                                               \
    void P##rms_norm(const float* x, const float* w, int rows, int D, float eps, float* y);\
    void P##fused_adaln(const float* x, const float* scale, const float* shift, int B,     \
                        int S, int D, float eps, float* y);                                 \
    void P##head_rms_norm(const float* x, const float* w, int N, int H, int Dh, float eps, \
                          float* y);                                                        \
    void P##rope_half(const float* x, const float* cos_t, const float* sin_t, int B,       \
                      int S, int H, int Dh, float* y);                                      \
    void P##rope_full(const float* x, const float* cos_t, const float* sin_t, int B,       \
                      int S, int H, int Dh, float* y);                                      \
    void P##sdpa(const float* q, const float* k, const float* v, const float* mask, int B, \
                 int H, int Sq, int Skv, int Dh, float scale, float* out);                  \
    void P##cond_module(const orc_cfg* c, const orc_io* io, const float* t, int B,         \
                        float* cond_out);                                                   \
    void P##adaln_vectors(const orc_cfg* c, const orc_block* blk, int which,               \
                          const float* cond, int B, float* shift, float* scale,            \
                          float* gate);                                                     \
    void P##gemm_fp8(const float* x, const float* w, int M, int K, int N, float* y);      \
    void P##conv1d(const float* x, int C, int L, const float* w, const float* b, int O,    \
                   int k, int dil, int pad, float* y);                                      \
    void P##conv_transpose1d(const float* x, int C, int L, const float* w, const float* b, \
                             int O, int k, int stride, int pad, int pad_out, float* y);     \
    void P##snake(const float* x, const float* alpha, int C, int L, float* y);             \
    void P##codec_decode(const orc_codec* cd, int B, int T, const float* latent, float* wav); \
    void P##text_block(const orc_enc_cfg* c, const orc_enc_block* blk, float* x,           \
                       const uint8_t* mask, int B, int S, const float* cos_t,              \
                       const float* sin_t);                                                 \
    void P##encoder_forward(const orc_enc_cfg* c, const orc_enc_block* blocks,             \
                            const float* embedding, const float* in_w, const float* in_b,  \
                            int in_dim, const float* out_norm, int mean_token, int B,       \
                            int S, const int32_t* ids, const float* latent,                \
                            const uint8_t* mask, float* out, uint8_t* mask_out);           \
    void P##swiglu(const float* h, const float* w13, const float* w2, int M, int D, int F, \
                   float* out);                                                             \
    void P##joint_attention(const orc_cfg* c, const orc_block* blk, const float* h, int B, \
                            int S, int T, const float* ctx_k, const float* ctx_v,          \
                            const uint8_t* ctx_mask, const uint8_t* lat_mask,              \
                            const float* cos_t, const float* sin_t, float* out);            \
    void P##block_forward(const orc_cfg* c, const orc_block* blk, float* x,                \
                          const float* cond, int B, int S, int T, const float* ctx_k,      \
                          const float* ctx_v, const uint8_t* ctx_mask,                      \
                          const uint8_t* lat_mask, const float* cos_t, const float* sin_t); \
    void P##forward(const orc_cfg* c, const orc_io* io, const orc_block* blocks, int B,    \
                    int S, const float* x_t, const float* t, int T, const float* ctx_k,    \
                    const float* ctx_v, const uint8_t* ctx_mask, const uint8_t* lat_mask,  \
                    float* v_out, float* debug);                                            \
    void P##build_kv_cache(const orc_cfg* c, const float* k_norm, int B, const float* text,\
                           const uint8_t* text_mask, int Tt, int Dt, const float* wk_text,  \
                           const float* wv_text, const float* aux, const uint8_t* aux_mask,\
                           int Ta, int Da, const float* wk_aux, const float* wv_aux,       \
                           float* ctx_k, float* ctx_v, uint8_t* ctx_mask);                  \
    int P##sample_joint_cfg(const orc_cfg* c, const orc_io* io, const orc_block* blocks,   \
                            int U, int S, const float* x0, int T, const float* ctx_k_cond, \
                            const float* ctx_v_cond, const uint8_t* mask_cond,             \
                            const float* ctx_k_unc, const float* ctx_v_unc,                \
                            const uint8_t* mask_unc, const uint8_t* lat_mask,              \
                            int num_steps, float scale, float min_t, float max_t,          \
                            int max_steps_run, float* x_out);                              \
    int P##sample_rf(const orc_cfg* c, const orc_io* io, const orc_block* blocks, int U,   \
                     int S, const float* x0, int T, const float* ctx_k, const float* ctx_v,\
                     const uint8_t* ctx_mask, const uint8_t* lat_mask,                      \
                     const orc_sampler* sp, int max_steps_run, float* x_out);

ORC_DECLARE(orc_f32_)
ORC_DECLARE(orc_f64_)

#ifdef __cplusplus
}
#endif
#endif
