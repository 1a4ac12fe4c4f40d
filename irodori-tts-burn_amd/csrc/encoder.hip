// Condition encoders on the GPU (irodori_encoder_*): TextEncoder / ReferenceLatentEncoder
// (text_encoder.rs:17-148, speaker_encoder.rs:85-162) with the conditioner norm and the
// speaker's masked-mean token (aux_conditioner.rs:60-85, :150-185).
//
// Per TextBlock, over the rows of a batch (M = batch * seq tokens):
//   h = RMSNorm(x, attn_norm)                      rmsnorm_w_kernel -> h (compute dtype)
//   [q|k|v|g] = h @ [Wq|Wk|Wv|Wg]                  one GEMM, f32 out
//   q, k head-normed + full RoPE, v, sigmoid(g)    enc_head_prep_kernel
//   o = SDPA(q, k, v, key mask) * sigmoid(g)       attn_kernel (head_dim 64 / 128)
//   x += o @ Wo                                    GEMM EPI_ADD
//   h = RMSNorm(x, mlp_norm); u = silu(h W1) h W3  GEMM EPI_SWIGLU
//   x = (x + u @ W2) * mask                        GEMM EPI_ADD with the row mask
// The front end writes x (masked) and the conditioner norm writes the state rows.
#include <memory>
#include <vector>

#include "../../include/irodori_hip.h"
#include "common.hpp"
#include "host.hpp"
#include "kernels.hpp"

using namespace irodori;

namespace {

struct EncLayer {
    void* w_qkvg = nullptr;  // [4E, E] rows Wq | Wk | Wv | W_gate (K-major)
    void* w_o = nullptr;     // [E, E]
    void* w13 = nullptr;     // [2F, E], W1 / W3 rows interleaved per 32
    void* w2 = nullptr;      // [E, F]
    float *attn_norm = nullptr, *mlp_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    bool loaded = false;
};

}  // namespace

struct irodori_encoder {
    int device = 0;
    irodori_encoder_config cfg{};
    bool bf16 = true;
    size_t esz = 2;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;
    uint64_t dev_bytes = 0;  // persistent device bytes held (tracked_alloc)
    std::vector<EncLayer> layers;
    float *embedding = nullptr, *in_w = nullptr, *in_b = nullptr, *out_norm = nullptr;
    bool io_loaded = false;
    // work buffers for max_rows * max_seq tokens
    float* x = nullptr;      // [M, E] residual stream
    void* h = nullptr;       // [M, E] normed GEMM input
    float* qkvg = nullptr;   // [M, 4E] projection
    void *q = nullptr, *k = nullptr, *v = nullptr;  // [B, H, S, Dh]
    void* gate = nullptr;    // [M, E]
    void* o = nullptr;       // [M, E] gated attention output
    void* u = nullptr;       // [M, F]
    float* mask = nullptr;   // [M] 1 / 0
    int* ids = nullptr;      // [M]
    float* lat = nullptr;    // [M, in_dim]
    float* out = nullptr;    // [B, S + 1, E]
    uint8_t* mask_out = nullptr;  // [B, S + 1]
    float *cs = nullptr, *sn = nullptr;  // RoPE [max_seq, Dh / 2]
};

namespace {

int enc_alloc(irodori_encoder* e, void** p, size_t bytes) { return tracked_alloc(e->allocs, e->dev_bytes, p, bytes); }
template <typename P>
int enc_alloc_t(irodori_encoder* e, P** p, size_t bytes) {
    return enc_alloc(e, reinterpret_cast<void**>(p), bytes);
}

int enc_upload(irodori_encoder* e, void* dst, const void* src, size_t bytes) {
    IRO_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, e->stream));
    return IRODORI_OK;
}

// Host f32 Burn [K, N] -> device K-major [N, K] in the compute dtype at dst (mode 1: the
// SwiGLU interleave).  Synchronous.
int enc_ingest(irodori_encoder* e, const float* host, int K, int N, int mode, void* dst) {
    float* stage = nullptr;
    const size_t bytes = sizeof(float) * (size_t)K * N;
    IRO_HIP_CHECK(hipMalloc(&stage, bytes));
    hipError_t err = hipMemcpyAsync(stage, host, bytes, hipMemcpyHostToDevice, e->stream);
    if (err == hipSuccess) {
        if (e->bf16)
            launch_transpose<bf16>(stage, K, N, mode, static_cast<bf16*>(dst), e->stream);
        else
            launch_transpose<float>(stage, K, N, mode, static_cast<float*>(dst), e->stream);
        err = hipGetLastError();
    }
    hipError_t e2 = hipStreamSynchronize(e->stream);
    (void)hipFree(stage);
    if (err == hipSuccess) err = e2;
    if (err != hipSuccess) {
        set_last_error(std::string("encoder weight ingest: ") + hipGetErrorString(err));
        return IRODORI_ERR_HIP;
    }
    return IRODORI_OK;
}

template <typename T>
int enc_gemm(irodori_encoder* e, int epi, const T* A, const void* W, int M, int N, int K, float* C, float* x,
             const float* rmask, T* U) {
    GemmArgs<T> ga{};
    ga.A = A;
    ga.W = static_cast<const T*>(W);
    ga.M = M;
    ga.N = N;
    ga.K = K;
    ga.S = M;
    ga.C = C;
    ga.x = x;
    ga.rmask = rmask;
    ga.U = U;
    if (launch_gemm<T>(epi, ga, e->stream)) {
        set_last_error("encoder gemm rejected the shape");
        return IRODORI_ERR_SHAPE;
    }
    return IRODORI_OK;
}

// One TextBlock over B rows of S tokens (see the file comment).
template <typename T>
int enc_block(irodori_encoder* e, const EncLayer& L, int B, int S) {
    const auto& g = e->cfg;
    const int E = g.dim, H = g.num_heads, Dh = E / H, F = g.mlp_hidden, M = B * S;
    T* h = static_cast<T*>(e->h);
    launch_rmsnorm_w<T>(e->x, L.attn_norm, M, E, g.norm_eps, h, E, e->stream);
    IRO_TRY(enc_gemm<T>(e, EPI_STORE, h, L.w_qkvg, M, 4 * E, E, e->qkvg, nullptr, nullptr, nullptr));
    launch_enc_head_prep<T>(e->qkvg, L.q_norm, L.k_norm, e->cs, e->sn, M, S, H, Dh, g.norm_eps,
                            static_cast<T*>(e->q), static_cast<T*>(e->k), static_cast<T*>(e->v),
                            static_cast<T*>(e->gate), e->stream);
    AttnArgs<T> aa{};
    aa.Q = static_cast<const T*>(e->q);
    aa.K0 = static_cast<const T*>(e->k);
    aa.V0 = static_cast<const T*>(e->v);
    aa.len0 = S;
    aa.stride0 = S;
    aa.mask0 = e->mask;
    aa.B = B;
    aa.H = H;
    aa.Sq = S;
    aa.scale = 1.0f / sqrtf((float)Dh);
    aa.out_mode = 0;
    aa.G = static_cast<const T*>(e->gate);
    aa.O = static_cast<T*>(e->o);
    const int arc = Dh == 64 ? launch_attention<T, 64>(aa, e->stream) : launch_attention<T, 128>(aa, e->stream);
    IRO_REQUIRE(arc == 0, IRODORI_ERR_SHAPE, "encoder attention rejected the shape");
    IRO_TRY(enc_gemm<T>(e, EPI_ADD, static_cast<const T*>(e->o), L.w_o, M, E, E, nullptr, e->x, nullptr, nullptr));
    launch_rmsnorm_w<T>(e->x, L.mlp_norm, M, E, g.norm_eps, h, E, e->stream);
    IRO_TRY(enc_gemm<T>(e, EPI_SWIGLU, h, L.w13, M, 2 * F, E, nullptr, nullptr, nullptr, static_cast<T*>(e->u)));
    IRO_TRY(enc_gemm<T>(e, EPI_ADD, static_cast<const T*>(e->u), L.w2, M, E, F, nullptr, e->x, e->mask, nullptr));
    return check_launch("encoder block");
}

}  // namespace

extern "C" {

int irodori_encoder_destroy(irodori_encoder* e) {
    if (!e) return IRODORI_OK;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    for (void* p : e->allocs) (void)hipFree(p);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
    return IRODORI_OK;
}

int irodori_encoder_create(int device, const irodori_encoder_config* cfg, irodori_encoder** out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(cfg && out, IRODORI_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    const irodori_encoder_config& g = *cfg;
    IRO_REQUIRE(g.compute_dtype == IRODORI_DTYPE_BF16 || g.compute_dtype == IRODORI_DTYPE_F32, IRODORI_ERR_DTYPE,
                "encoder compute_dtype must be IRODORI_DTYPE_BF16 or IRODORI_DTYPE_F32");
    IRO_REQUIRE(g.dim > 0 && g.num_layers >= 0 && g.num_heads > 0 && g.dim % g.num_heads == 0, IRODORI_ERR_SHAPE,
                "dim must be a positive multiple of num_heads");
    const int Dh = g.dim / (g.num_heads > 0 ? g.num_heads : 1);
    IRO_REQUIRE(Dh == 64 || Dh == 128, IRODORI_ERR_SHAPE, "encoder head_dim must be 64 or 128");
    IRO_REQUIRE(g.dim % 128 == 0, IRODORI_ERR_SHAPE, "encoder dim must be a multiple of 128");
    IRO_REQUIRE(g.mlp_hidden > 0 && g.mlp_hidden % 64 == 0, IRODORI_ERR_SHAPE,
                "encoder mlp_hidden must be a positive multiple of 64");
    IRO_REQUIRE((g.vocab_size > 0) != (g.in_dim > 0), IRODORI_ERR_CONFIG,
                "exactly one of vocab_size (tokens) and in_dim (latent frames) must be set");
    IRO_REQUIRE(g.mean_token == 0 || g.mean_token == 1, IRODORI_ERR_CONFIG, "mean_token must be 0 or 1");
    IRO_REQUIRE(g.norm_eps > 0.f && std::isfinite(g.norm_eps), IRODORI_ERR_CONFIG, "norm_eps must be > 0");
    IRO_REQUIRE(g.max_rows > 0 && g.max_seq > 0, IRODORI_ERR_SHAPE, "max sizes must be positive");
    int ndev = 0;
    hipError_t err = hipGetDeviceCount(&ndev);
    IRO_REQUIRE(err == hipSuccess && ndev > 0, IRODORI_ERR_HIP, "no HIP device available");
    IRO_REQUIRE(device >= 0 && device < ndev, IRODORI_ERR_INVALID_ARG, "device index out of range");
    IRO_HIP_CHECK(hipSetDevice(device));

    std::unique_ptr<irodori_encoder, int (*)(irodori_encoder*)> e(new irodori_encoder(), irodori_encoder_destroy);
    e->device = device;
    e->cfg = g;
    e->bf16 = g.compute_dtype == IRODORI_DTYPE_BF16;
    e->esz = e->bf16 ? 2 : 4;
    IRO_HIP_CHECK(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
    const size_t E = g.dim, F = g.mlp_hidden, M = (size_t)g.max_rows * g.max_seq, es = e->esz;
    e->layers.resize(g.num_layers);
    for (auto& L : e->layers) {
        IRO_TRY(enc_alloc(e.get(), &L.w_qkvg, es * 4 * E * E));
        IRO_TRY(enc_alloc(e.get(), &L.w_o, es * E * E));
        IRO_TRY(enc_alloc(e.get(), &L.w13, es * 2 * F * E));
        IRO_TRY(enc_alloc(e.get(), &L.w2, es * E * F));
        IRO_TRY(enc_alloc_t(e.get(), &L.attn_norm, sizeof(float) * E));
        IRO_TRY(enc_alloc_t(e.get(), &L.mlp_norm, sizeof(float) * E));
        IRO_TRY(enc_alloc_t(e.get(), &L.q_norm, sizeof(float) * E));
        IRO_TRY(enc_alloc_t(e.get(), &L.k_norm, sizeof(float) * E));
    }
    if (g.vocab_size > 0) IRO_TRY(enc_alloc_t(e.get(), &e->embedding, sizeof(float) * (size_t)g.vocab_size * E));
    if (g.in_dim > 0) {
        IRO_TRY(enc_alloc_t(e.get(), &e->in_w, sizeof(float) * (size_t)g.in_dim * E));
        IRO_TRY(enc_alloc_t(e.get(), &e->in_b, sizeof(float) * E));
        IRO_TRY(enc_alloc_t(e.get(), &e->lat, sizeof(float) * M * g.in_dim));
    }
    IRO_TRY(enc_alloc_t(e.get(), &e->out_norm, sizeof(float) * E));
    IRO_TRY(enc_alloc_t(e.get(), &e->x, sizeof(float) * M * E));
    IRO_TRY(enc_alloc(e.get(), &e->h, es * M * E));
    IRO_TRY(enc_alloc_t(e.get(), &e->qkvg, sizeof(float) * M * 4 * E));
    IRO_TRY(enc_alloc(e.get(), &e->q, es * M * E));
    IRO_TRY(enc_alloc(e.get(), &e->k, es * M * E));
    IRO_TRY(enc_alloc(e.get(), &e->v, es * M * E));
    IRO_TRY(enc_alloc(e.get(), &e->gate, es * M * E));
    IRO_TRY(enc_alloc(e.get(), &e->o, es * M * E));
    IRO_TRY(enc_alloc(e.get(), &e->u, es * M * F));
    IRO_TRY(enc_alloc_t(e.get(), &e->mask, sizeof(float) * M));
    IRO_TRY(enc_alloc_t(e.get(), &e->ids, sizeof(int) * M));
    IRO_TRY(enc_alloc_t(e.get(), &e->out, sizeof(float) * (size_t)g.max_rows * (g.max_seq + 1) * E));
    IRO_TRY(enc_alloc_t(e.get(), &e->mask_out, (size_t)g.max_rows * (g.max_seq + 1)));
    std::vector<float> cs, sn;
    host_rope_tables(g.max_seq, Dh, 10000.f, cs, sn);  // precompute_rope_freqs(head_dim, seq, 1e4)
    IRO_TRY(enc_alloc_t(e.get(), &e->cs, sizeof(float) * cs.size()));
    IRO_TRY(enc_alloc_t(e.get(), &e->sn, sizeof(float) * sn.size()));
    IRO_TRY(enc_upload(e.get(), e->cs, cs.data(), sizeof(float) * cs.size()));
    IRO_TRY(enc_upload(e.get(), e->sn, sn.data(), sizeof(float) * sn.size()));
    IRO_HIP_CHECK(hipStreamSynchronize(e->stream));
    *out = e.release();
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_encoder_load_io_weights(irodori_encoder* e, const irodori_encoder_io_weights* w) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(e && w && w->out_norm, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = e->cfg;
    IRO_REQUIRE(g.vocab_size == 0 || w->embedding, IRODORI_ERR_INVALID_ARG, "null embedding");
    IRO_REQUIRE(g.in_dim == 0 || (w->in_w && w->in_b), IRODORI_ERR_INVALID_ARG, "null in_proj weights");
    IRO_HIP_CHECK(hipSetDevice(e->device));
    const size_t E = g.dim;
    if (g.vocab_size > 0) IRO_TRY(enc_upload(e, e->embedding, w->embedding, sizeof(float) * g.vocab_size * E));
    if (g.in_dim > 0) {
        IRO_TRY(enc_upload(e, e->in_w, w->in_w, sizeof(float) * g.in_dim * E));
        IRO_TRY(enc_upload(e, e->in_b, w->in_b, sizeof(float) * E));
    }
    IRO_TRY(enc_upload(e, e->out_norm, w->out_norm, sizeof(float) * E));
    IRO_HIP_CHECK(hipStreamSynchronize(e->stream));
    e->io_loaded = true;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_encoder_load_block_weights(irodori_encoder* e, int layer, const irodori_encoder_block_weights* w) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(e && w, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(layer >= 0 && layer < e->cfg.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(w->attn_norm && w->wq && w->wk && w->wv && w->wo && w->w_gate && w->q_norm && w->k_norm &&
                    w->mlp_norm && w->w13 && w->w2,
                IRODORI_ERR_INVALID_ARG, "null block weight pointer");
    IRO_HIP_CHECK(hipSetDevice(e->device));
    const int E = e->cfg.dim, F = e->cfg.mlp_hidden;
    auto& L = e->layers[layer];
    char* qkvg = static_cast<char*>(L.w_qkvg);
    const size_t rows = e->esz * (size_t)E * E;  // one E-row block of the fused weight
    IRO_TRY(enc_ingest(e, w->wq, E, E, 0, qkvg));
    IRO_TRY(enc_ingest(e, w->wk, E, E, 0, qkvg + rows));
    IRO_TRY(enc_ingest(e, w->wv, E, E, 0, qkvg + 2 * rows));
    IRO_TRY(enc_ingest(e, w->w_gate, E, E, 0, qkvg + 3 * rows));
    IRO_TRY(enc_ingest(e, w->wo, E, E, 0, L.w_o));
    IRO_TRY(enc_ingest(e, w->w13, E, 2 * F, 1, L.w13));
    IRO_TRY(enc_ingest(e, w->w2, F, E, 0, L.w2));
    IRO_TRY(enc_upload(e, L.attn_norm, w->attn_norm, sizeof(float) * E));
    IRO_TRY(enc_upload(e, L.mlp_norm, w->mlp_norm, sizeof(float) * E));
    IRO_TRY(enc_upload(e, L.q_norm, w->q_norm, sizeof(float) * E));
    IRO_TRY(enc_upload(e, L.k_norm, w->k_norm, sizeof(float) * E));
    IRO_HIP_CHECK(hipStreamSynchronize(e->stream));
    L.loaded = true;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_encoder_forward(irodori_encoder* e, int B, int S, const int32_t* ids, const float* latent,
                            const uint8_t* mask, float* state_out, uint8_t* mask_out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(e && mask && state_out, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = e->cfg;
    IRO_REQUIRE(B > 0 && B <= g.max_rows && S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE,
                "batch / seq out of range [1, max_rows] x [1, max_seq]");
    IRO_REQUIRE(g.vocab_size == 0 || ids, IRODORI_ERR_INVALID_ARG, "token encoder needs ids");
    IRO_REQUIRE(g.in_dim == 0 || latent, IRODORI_ERR_INVALID_ARG, "latent encoder needs latent frames");
    IRO_REQUIRE(e->io_loaded, IRODORI_ERR_NOT_LOADED, "encoder io weights not loaded");
    for (int l = 0; l < g.num_layers; l++)
        IRO_REQUIRE(e->layers[l].loaded, IRODORI_ERR_NOT_LOADED,
                    "encoder block " + std::to_string(l) + " weights not loaded");
    const int M = B * S, E = g.dim, T = S + g.mean_token;
    if (ids)
        for (int i = 0; i < M && g.vocab_size > 0; i++)
            IRO_REQUIRE(ids[i] >= 0 && ids[i] < g.vocab_size, IRODORI_ERR_INVALID_ARG, "token id out of range");
    IRO_HIP_CHECK(hipSetDevice(e->device));
    std::vector<float> mf(M);
    for (int i = 0; i < M; i++) mf[i] = mask[i] ? 1.f : 0.f;
    IRO_TRY(enc_upload(e, e->mask, mf.data(), sizeof(float) * M));
    if (g.vocab_size > 0) {
        IRO_TRY(enc_upload(e, e->ids, ids, sizeof(int) * M));
        launch_enc_embed(e->ids, e->embedding, e->mask, e->x, M, E, e->stream);
    } else {
        IRO_TRY(enc_upload(e, e->lat, latent, sizeof(float) * (size_t)M * g.in_dim));
        launch_enc_inproj(e->lat, e->in_w, e->in_b, e->mask, e->x, M, g.in_dim, E, e->stream);
    }
    for (int l = 0; l < g.num_layers; l++)
        IRO_TRY(e->bf16 ? enc_block<bf16>(e, e->layers[l], B, S) : enc_block<float>(e, e->layers[l], B, S));
    // Conditioner norm into the state rows (after the mean token's slot), then the token.
    for (int b = 0; b < B; b++)
        launch_rmsnorm_w<float>(e->x + (size_t)b * S * E, e->out_norm, S, E, g.norm_eps,
                                e->out + ((size_t)b * T + g.mean_token) * E, E, e->stream);
    if (g.mean_token) launch_enc_mean_token(e->out, e->mask, e->mask_out, B, S, E, e->stream);
    IRO_TRY(check_launch("encoder output"));
    IRO_HIP_CHECK(hipMemcpyAsync(state_out, e->out, sizeof(float) * (size_t)B * T * E, hipMemcpyDeviceToHost,
                                 e->stream));
    if (mask_out && g.mean_token)
        IRO_HIP_CHECK(hipMemcpyAsync(mask_out, e->mask_out, (size_t)B * T, hipMemcpyDeviceToHost, e->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(e->stream));
    if (mask_out)
        for (int b = 0; b < B; b++)
            for (int s = 0; s < S; s++) mask_out[(size_t)b * T + g.mean_token + s] = mask[(size_t)b * S + s] ? 1 : 0;
    return IRODORI_OK;
    IRO_GUARD_END
}

}  // extern "C"
