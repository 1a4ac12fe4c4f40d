// DACVAE decoder on the GPU (irodori_codec_*): DacVaeCodec::decode (codec/model.rs:60-65)
// = quantizer.out_proj (bottleneck.rs:21-23), the decoder stem, the DecoderBlocks and the
// watermark head (decoder.rs), with the weights of codec/weights.rs:225-292.
//
// Layout: every activation is channels-last [frames, Cp] (one GEMM row per frame; Cp the
// channel count rounded up to 64 with the extra channels exactly zero: their weights,
// biases and Snake alphas are zero).  The residual stream x is f32; the GEMM operands are
// in the compute dtype, with `kHalo` zero rows on both sides where a convolution reads
// them (its zero padding).  Per utterance row:
//   s = out_proj(latent)                     codec_in_kernel        -> S  [T + 2h, Pp]
//   x = stem(s)     (k 7, pad 3)             conv GEMM EPI_STORE    -> X  [T, Dp]
//   per DecoderBlock (rate r, C -> O = C / 2):
//     x = ConvTranspose1d(Snake(x)) (k 2r)   conv GEMM EPI_STORE    -> X  (see below)
//     per ResidualUnit (dilation 1, 3, 9), Op = 64 / 128 / 192 channels:
//       x += conv_1x1(Snake(conv_k7(Snake(x)) + b)) + b   conv GEMM EPI_RESUNIT
//     wider streams (two kernels):
//       s2 = Snake(conv_k7(Snake(x)) + b)    conv GEMM EPI_SNAKE    -> S2 [L, Op]
//       x += conv_1x1(s2) + b                GEMM EPI_ADD
//   wav = tanh(head_conv_k7(Snake(x)))       codec_head_kernel
// A Snake of x that feeds a convolution is written by the epilogue producing x (the stem,
// the transposed convolution, the 1x1 residual add) into the haloed operand S / S3.
//
// ConvTranspose1d(stride r, kernel 2r, padding ceil(r/2), output padding r % 2) as one
// GEMM: output frame t with t + pad = i r + q (0 <= q < r) sums input frame i through tap
// q and input frame i - 1 through tap q + r.  So the GEMM row i (0 <= i <= L) takes the
// two-tap window [x[i-1], x[i]] (an implicit im2col with 2 taps) and its N = r * Op
// columns (q, o) are output frames i r + q - pad: the [L + 1, r Op] result read as
// [(L + 1) r, Op] rows is the transposed convolution's output shifted by pad rows, so the
// next stage's x starts pad rows into the same buffer and no scatter pass is needed.
#include <algorithm>
#include <memory>
#include <vector>

#include "../../include/irodori_hip.h"
#include "common.hpp"
#include "host.hpp"
#include "kernels.hpp"

using namespace irodori;

namespace {

constexpr int kHalo = 32;  // >= the widest padding: 3 * dilation 9 = 27
constexpr int kDil[3] = {1, 3, 9};

inline int round64(int c) { return (c + 63) / 64 * 64; }
inline int round_to(int v, int m) { return (v + m - 1) / m * m; }
// Channels of a stream on the device: 65..96 stay at 96 (one tile column of the 96-wide
// tiles, K slices straddling taps), everything else rounds up to 64.
inline int pad_channels(int c) { return c > 64 && c <= 96 ? 96 : round64(c); }
// Streams whose ResidualUnits run as one kernel (EPI_RESUNIT: every channel in one tile).
inline bool fused_width(int cp) { return cp == 64 || cp == 96 || cp == 128 || cp == 192; }

struct CodecBlock {
    int cin = 0, cout = 0, cin_p = 0, cout_p = 0, rate = 0;
    float* alpha = nullptr;  // Snake constants [3, cin_p] (snake_consts)
    void* wt = nullptr;      // [rate * cout_p, 2 * cin_p]: row (q, o), k (tap window, c)
    float* bt = nullptr;     // [rate * cout_p] bias per (q, o)
    float* ra0[3] = {};      // [3, cout_p]
    void* rw[3] = {};        // [cout_p, 7 * cout_p]
    float* rb[3] = {};       // [cout_p] or null
    float* ra1[3] = {};
    void* pw[3] = {};        // [cout_p, cout_p]
    float* pb[3] = {};
};

}  // namespace

struct irodori_codec {
    int device = 0;
    irodori_codec_config cfg{};
    bool bf16 = true;
    size_t esz = 2;
    int hop = 1, proj_p = 0, dim_p = 0, last_p = 0;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;
    uint64_t dev_bytes = 0;  // persistent device bytes held (tracked_alloc)
    float *in_w = nullptr, *in_b = nullptr;  // [proj_p, latent_dim], [proj_p]
    void* stem_w = nullptr;                  // [dim_p, 7 * proj_p]
    float* stem_b = nullptr;                 // [dim_p] or null
    std::vector<CodecBlock> blocks;
    float *head_alpha = nullptr, *head_w = nullptr, *head_b = nullptr;  // [3, last_p], [7, last_p], [1]
    bool loaded = false;
    size_t x_elems = 0, s_elems = 0, s2_elems = 0;
    float* X = nullptr;  // residual stream (and the transposed convolutions' output)
    void* S = nullptr;   // haloed convolution operand
    void* S3 = nullptr;  // the other haloed operand (S and S3 alternate)
    void* S2 = nullptr;  // the 1x1 convolutions' operand
    float* lat = nullptr;  // [max_frames, latent_dim] staging of the host entry point
    float* wav = nullptr;  // [max_frames * hop]
};

namespace {

int codec_alloc(irodori_codec* c, void** p, size_t bytes) { return tracked_alloc(c->allocs, c->dev_bytes, p, bytes); }
template <typename P>
int codec_alloc_t(irodori_codec* c, P** p, size_t bytes) {
    return codec_alloc(c, reinterpret_cast<void**>(p), bytes);
}

// Host f32 -> device f32 (synchronous).
int put_f32(irodori_codec* c, float* dst, const std::vector<float>& v) {
    IRO_HIP_CHECK(hipMemcpyAsync(dst, v.data(), sizeof(float) * v.size(), hipMemcpyHostToDevice, c->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    return IRODORI_OK;
}

// Host f32 -> device operand in the compute dtype (synchronous).
int put_operand(irodori_codec* c, void* dst, const std::vector<float>& v) {
    if (!c->bf16) return put_f32(c, static_cast<float*>(dst), v);
    float* stage = nullptr;
    IRO_HIP_CHECK(hipMalloc(&stage, sizeof(float) * v.size()));
    hipError_t err = hipMemcpyAsync(stage, v.data(), sizeof(float) * v.size(), hipMemcpyHostToDevice, c->stream);
    if (err == hipSuccess) {
        launch_cvt_f32<bf16>(stage, (long)v.size(), static_cast<bf16*>(dst), c->stream);
        err = hipGetLastError();
    }
    hipError_t e2 = hipStreamSynchronize(c->stream);
    (void)hipFree(stage);
    if (err == hipSuccess) err = e2;
    if (err != hipSuccess) {
        set_last_error(std::string("codec weight ingest: ") + hipGetErrorString(err));
        return IRODORI_ERR_HIP;
    }
    return IRODORI_OK;
}

// Burn Conv1d weight [O, C, k] -> K-major [Op, Kp]: row o, column j * Cp + c, zero past
// k * Cp (Kp: the taps' span rounded up to whole GEMM slices).
std::vector<float> conv_rows(const float* w, int O, int C, int k, int Op, int Cp, int Kp) {
    std::vector<float> out((size_t)Op * Kp, 0.f);
    for (int o = 0; o < O; o++)
        for (int c = 0; c < C; c++)
            for (int j = 0; j < k; j++) out[(size_t)o * Kp + (size_t)j * Cp + c] = w[((size_t)o * C + c) * k + j];
    return out;
}

// Burn ConvTranspose1d weight [C, O, 2r] -> [r * Op, 2 * Cp]: row (q, o); window slot 0
// (input frame i - 1) takes tap q + r, slot 1 (frame i) tap q.
std::vector<float> convt_rows(const float* w, int C, int O, int r, int Cp, int Op) {
    std::vector<float> out((size_t)r * Op * 2 * Cp, 0.f);
    for (int q = 0; q < r; q++)
        for (int o = 0; o < O; o++) {
            float* row = out.data() + ((size_t)q * Op + o) * 2 * Cp;
            for (int c = 0; c < C; c++) {
                const float* wc = w + ((size_t)c * O + o) * 2 * r;
                row[c] = wc[q + r];
                row[Cp + c] = wc[q];
            }
        }
    return out;
}

// Snake constants of a channel vector a [n], padded to np: the block [3, np] = (a, a / pi,
// 0.5 / (a + 1e-9)) in f32, all zero past n (a padded channel carries exact zeros).
std::vector<float> snake_consts(const float* a, int n, int np) {
    std::vector<float> out((size_t)3 * np, 0.f);
    for (int i = 0; i < n; i++) {
        out[i] = a[i];
        out[np + i] = a[i] / 3.14159265358979f;
        out[2 * np + i] = 0.5f / (a[i] + 1e-9f);
    }
    return out;
}

// A per-channel vector padded with zeros to np entries, repeated `rep` times.
std::vector<float> padded(const float* v, int n, int np, int rep = 1) {
    std::vector<float> out((size_t)np * rep, 0.f);
    if (v)
        for (int r = 0; r < rep; r++)
            for (int i = 0; i < n; i++) out[(size_t)r * np + i] = v[i];
    return out;
}

// One convolution GEMM.  `cp` > 0: implicit im2col over taps = K / cp source rows spaced
// `dil` (launch_gemm_conv); 0: a plain GEMM (the 1x1 convolutions).  `U` (with its Snake
// constants `alpha` of alpha_n channels and the window [u_lo, u_hi) of linear output
// indices) receives Snake(output) for the next convolution.
template <typename T>
struct ConvCall {
    int epi = EPI_STORE;
    const T* A = nullptr;
    int cp = 0, dil = 1, rows = 0, M = 0, N = 0, K = 0;
    const void* W = nullptr;
    const float* bias = nullptr;
    const float* alpha = nullptr;
    int alpha_n = 0;
    float* C = nullptr;
    T* U = nullptr;
    long u_lo = 0, u_hi = 0;
    const void* W2 = nullptr;  // EPI_RESUNIT: the 1x1 conv [N, N], its bias, the next Snake
    const float* bias2 = nullptr;
    const float* alpha2 = nullptr;
};

template <typename T>
int codec_conv(const ConvCall<T>& k, hipStream_t st) {
    GemmArgs<T> ga{};
    ga.A = k.A;
    ga.W = static_cast<const T*>(k.W);
    ga.M = k.M;
    ga.N = k.N;
    ga.K = k.K;
    ga.S = k.M;
    ga.C = k.C;
    ga.x = k.C;
    ga.U = k.U;
    ga.bias = k.bias;
    ga.alpha = k.alpha;
    ga.alpha_n = k.alpha_n;
    ga.u_lo = k.u_lo;
    ga.u_hi = k.u_hi;
    ga.W2 = static_cast<const T*>(k.W2);
    ga.bias2 = k.bias2;
    ga.alpha2 = k.alpha2;
    ga.conv_cp = k.cp;
    ga.conv_dil = k.dil;
    ga.conv_rows = k.rows;
    const int rc = k.cp > 0 ? launch_gemm_conv<T>(k.epi, ga, st) : launch_gemm<T>(k.epi, ga, st);
    if (rc) {
        set_last_error("codec convolution GEMM rejected the shape (M " + std::to_string(k.M) + ", N " +
                       std::to_string(k.N) + ", K " + std::to_string(k.K) + ")");
        return IRODORI_ERR_SHAPE;
    }
    return IRODORI_OK;
}

// One utterance row: lat [frames, latent_dim] -> wav [frames * hop], device pointers.
// Every Snake except the head's is applied in the epilogue of the GEMM that produces its
// input (stem, transposed convolution, 1x1 residual add), which writes the next
// convolution's haloed operand: two operand buffers alternate (a convolution never writes
// the buffer it reads), and each new operand layout gets its halo rows zeroed.
template <typename T>
int codec_row(irodori_codec* c, const float* lat, int frames, float* wav, hipStream_t st) {
    const auto& g = c->cfg;
    const int H = kHalo;
    T* cur = static_cast<T*>(c->S);
    T* nxt = static_cast<T*>(c->S3);
    T* S2 = static_cast<T*>(c->S2);
    launch_codec_in<T>(lat, frames, g.latent_dim, c->in_w, c->in_b, c->proj_p, H, cur, st);
    int L = frames;
    {  // stem; its epilogue writes Snake(x) of block 0's entry into nxt
        const CodecBlock& b0 = c->blocks[0];
        launch_codec_zero_halo<T>(nxt, L, c->dim_p, H, st);
        ConvCall<T> k;
        k.A = cur + (size_t)(H - 3) * c->proj_p;
        k.cp = c->proj_p;
        k.rows = L + H + 3;
        k.M = L;
        k.N = c->dim_p;
        k.K = 7 * c->proj_p;
        k.W = c->stem_w;
        k.bias = c->stem_b;
        k.C = c->X;
        k.U = nxt + (size_t)H * c->dim_p;
        k.alpha = b0.alpha;
        k.alpha_n = b0.cin_p;
        k.u_hi = (long)L * c->dim_p;
        IRO_TRY(codec_conv<T>(k, st));
        std::swap(cur, nxt);
    }
    float* x = c->X;
    for (size_t bi = 0; bi < c->blocks.size(); bi++) {
        const CodecBlock& b = c->blocks[bi];
        const int pad = (b.rate + 1) / 2, Op = b.cout_p, Lo = L * b.rate;
        {  // transposed convolution; the epilogue writes Snake(x) of unit 0 into nxt
            launch_codec_zero_halo<T>(nxt, Lo, Op, H, st);
            ConvCall<T> k;
            k.A = cur + (size_t)(H - 1) * b.cin_p;
            k.cp = b.cin_p;
            k.rows = L + H + 1;
            k.M = L + 1;
            k.N = b.rate * Op;
            k.K = 2 * b.cin_p;
            k.W = b.wt;
            k.bias = b.bt;
            k.C = c->X;
            // Row i, column (q, o) is frame i r + q - pad: the operand row frame + H.
            k.U = nxt + (size_t)(H - pad) * Op;
            k.alpha = b.ra0[0];
            k.alpha_n = Op;
            k.u_lo = (long)pad * Op;
            k.u_hi = (long)(pad + Lo) * Op;
            IRO_TRY(codec_conv<T>(k, st));
            std::swap(cur, nxt);
        }
        x = c->X + (size_t)pad * Op;
        L = Lo;
        // Streams of 64 / 128 / 192 channels fit one tile column: each ResidualUnit is one
        // kernel (EPI_RESUNIT), which writes the next Snake into the other operand buffer.
        const bool fused = fused_width(Op);
        const int K7 = round_to(7 * Op, 128 / (int)c->esz);
        if (fused) launch_codec_zero_halo<T>(nxt, L, Op, H, st);
        for (int u = 0; u < 3; u++) {
            const int d = kDil[u];
            const float* next_alpha = u < 2 ? b.ra0[u + 1] : bi + 1 < c->blocks.size() ? c->blocks[bi + 1].alpha : nullptr;
            if (fused) {
                ConvCall<T> k;
                k.epi = EPI_RESUNIT;
                k.A = cur + (size_t)(H - 3 * d) * Op;
                k.cp = Op;
                k.dil = d;
                k.rows = L + H + 3 * d;
                k.M = L;
                k.N = Op;
                k.K = K7;
                k.W = b.rw[u];
                k.bias = b.rb[u];
                k.alpha = b.ra1[u];
                k.alpha_n = Op;
                k.C = x;
                k.W2 = b.pw[u];
                k.bias2 = b.pb[u];
                if (next_alpha) {
                    k.U = nxt + (size_t)H * Op;
                    k.alpha2 = next_alpha;
                }
                IRO_TRY(codec_conv<T>(k, st));
                if (next_alpha) std::swap(cur, nxt);
                continue;
            }
            ConvCall<T> k7;
            k7.epi = EPI_SNAKE;
            k7.A = cur + (size_t)(H - 3 * d) * Op;
            k7.cp = Op;
            k7.dil = d;
            k7.rows = L + H + 3 * d;
            k7.M = L;
            k7.N = Op;
            k7.K = K7;
            k7.W = b.rw[u];
            k7.bias = b.rb[u];
            k7.alpha = b.ra1[u];
            k7.alpha_n = Op;
            k7.U = S2;
            IRO_TRY(codec_conv<T>(k7, st));
            ConvCall<T> k1;  // x += conv_1x1(s2) + b, and the next Snake of x into cur
            k1.epi = EPI_ADD;
            k1.A = S2;
            k1.M = L;
            k1.N = Op;
            k1.K = Op;
            k1.W = b.pw[u];
            k1.bias = b.pb[u];
            k1.C = x;
            if (next_alpha) {
                k1.U = cur + (size_t)H * Op;
                k1.alpha = next_alpha;
                k1.alpha_n = Op;
                k1.u_hi = (long)L * Op;
            }
            IRO_TRY(codec_conv<T>(k1, st));
        }
    }
    launch_codec_head<T>(x, L, c->last_p, c->head_alpha, c->head_w, c->head_b, wav, st);
    return check_launch("codec decode");
}

int codec_decode(irodori_codec* c, int B, int frames, const float* lat, float* wav, hipStream_t st) {
    const size_t per_lat = (size_t)frames * c->cfg.latent_dim, per_wav = (size_t)frames * c->hop;
    for (int b = 0; b < B; b++)
        IRO_TRY(c->bf16 ? codec_row<bf16>(c, lat + b * per_lat, frames, wav + b * per_wav, st)
                        : codec_row<float>(c, lat + b * per_lat, frames, wav + b * per_wav, st));
    return IRODORI_OK;
}

}  // namespace

extern "C" {

int irodori_codec_destroy(irodori_codec* c) {
    if (!c) return IRODORI_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (void* p : c->allocs) (void)hipFree(p);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return IRODORI_OK;
}

int irodori_codec_create(int device, const irodori_codec_config* cfg, irodori_codec** out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(cfg && out, IRODORI_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    const irodori_codec_config& g = *cfg;
    IRO_REQUIRE(g.compute_dtype == IRODORI_DTYPE_BF16 || g.compute_dtype == IRODORI_DTYPE_F32, IRODORI_ERR_DTYPE,
                "codec compute_dtype must be IRODORI_DTYPE_BF16 or IRODORI_DTYPE_F32");
    IRO_REQUIRE(g.num_blocks >= 1 && g.num_blocks <= IRODORI_CODEC_MAX_BLOCKS, IRODORI_ERR_CONFIG,
                "codec num_blocks must be in [1, 8]");
    IRO_REQUIRE(g.latent_dim > 0 && g.latent_dim <= 1024 && g.proj_dim > 0 && g.proj_dim % 8 == 0, IRODORI_ERR_SHAPE,
                "codec latent_dim must be in [1, 1024] and proj_dim a positive multiple of 8");
    IRO_REQUIRE(g.decoder_dim > 0 && g.decoder_dim % (8 << g.num_blocks) == 0, IRODORI_ERR_SHAPE,
                "codec decoder_dim must be a multiple of 8 * 2^num_blocks (the channels halve per block)");
    long hop = 1;
    for (int i = 0; i < g.num_blocks; i++) {
        IRO_REQUIRE(g.rates[i] >= 2 && g.rates[i] <= 64, IRODORI_ERR_CONFIG, "codec rates must be in [2, 64]");
        hop *= g.rates[i];
    }
    IRO_REQUIRE(g.max_frames > 0 && (long)g.max_frames * hop < (1L << 31), IRODORI_ERR_SHAPE,
                "codec max_frames must be positive and max_frames * hop below 2^31");
    int ndev = 0;
    hipError_t err = hipGetDeviceCount(&ndev);
    IRO_REQUIRE(err == hipSuccess && ndev > 0, IRODORI_ERR_HIP, "no HIP device available");
    IRO_REQUIRE(device >= 0 && device < ndev, IRODORI_ERR_INVALID_ARG, "device index out of range");
    IRO_HIP_CHECK(hipSetDevice(device));
    std::unique_ptr<irodori_codec, int (*)(irodori_codec*)> c(new irodori_codec(), irodori_codec_destroy);
    c->device = device;
    c->cfg = g;
    c->bf16 = g.compute_dtype == IRODORI_DTYPE_BF16;
    c->esz = c->bf16 ? 2 : 4;
    c->hop = (int)hop;
    c->proj_p = round64(g.proj_dim);
    c->dim_p = pad_channels(g.decoder_dim);
    IRO_HIP_CHECK(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    const size_t es = c->esz, H = kHalo;
    size_t L = g.max_frames;
    size_t xe = L * c->dim_p, se = (L + 2 * H) * c->proj_p, s2e = 0;
    int C = g.decoder_dim;
    c->blocks.resize(g.num_blocks);
    for (int i = 0; i < g.num_blocks; i++) {
        CodecBlock& b = c->blocks[i];
        b.cin = C;
        b.cout = C / 2;
        b.cin_p = pad_channels(b.cin);
        b.cout_p = pad_channels(b.cout);
        const int slice = 128 / (int)es;  // GEMM K slice in elements
        IRO_REQUIRE(b.cout_p % 64 == 0 || fused_width(b.cout_p), IRODORI_ERR_SHAPE, "codec stream width without a kernel");
        b.rate = g.rates[i];
        se = std::max(se, (L + 2 * H) * b.cin_p);
        xe = std::max(xe, (L + 1) * b.rate * b.cout_p);
        L *= b.rate;
        se = std::max(se, (L + 2 * H) * b.cout_p);
        s2e = std::max(s2e, L * b.cout_p);
        C = b.cout;
        IRO_TRY(codec_alloc_t(c.get(), &b.alpha, sizeof(float) * 3 * b.cin_p));
        IRO_TRY(codec_alloc(c.get(), &b.wt, es * b.rate * b.cout_p * 2 * b.cin_p));
        IRO_TRY(codec_alloc_t(c.get(), &b.bt, sizeof(float) * b.rate * b.cout_p));
        for (int u = 0; u < 3; u++) {
            IRO_TRY(codec_alloc_t(c.get(), &b.ra0[u], sizeof(float) * 3 * b.cout_p));
            IRO_TRY(codec_alloc_t(c.get(), &b.ra1[u], sizeof(float) * 3 * b.cout_p));
            IRO_TRY(codec_alloc(c.get(), &b.rw[u], es * b.cout_p * round_to(7 * b.cout_p, slice)));
            IRO_TRY(codec_alloc(c.get(), &b.pw[u], es * b.cout_p * round_to(b.cout_p, slice)));
        }
    }
    c->last_p = pad_channels(C);
    IRO_REQUIRE(c->last_p <= 256, IRODORI_ERR_SHAPE, "codec head width (decoder_dim >> num_blocks) must be at most 256");
    // The convolution GEMMs address each haloed operand [frames + 2 halo, channels] through one
    // 32-bit buffer resource, so the largest of them must stay below 4 GiB; rejected here,
    // before the work buffers are allocated, rather than at the first decode.
    IRO_REQUIRE(es * std::max(se, s2e) <= 0xffffffffull, IRODORI_ERR_SHAPE,
                "codec max_frames too large: the largest convolution operand would take " +
                    std::to_string(es * std::max(se, s2e)) + " bytes, above the 4 GiB a GEMM operand may span");
    c->x_elems = xe;
    c->s_elems = se;
    c->s2_elems = s2e;
    IRO_TRY(codec_alloc_t(c.get(), &c->in_w, sizeof(float) * c->proj_p * g.latent_dim));
    IRO_TRY(codec_alloc_t(c.get(), &c->in_b, sizeof(float) * c->proj_p));
    IRO_TRY(codec_alloc(c.get(), &c->stem_w, es * c->dim_p * 7 * c->proj_p));
    IRO_TRY(codec_alloc_t(c.get(), &c->head_alpha, sizeof(float) * 3 * c->last_p));
    IRO_TRY(codec_alloc_t(c.get(), &c->head_w, sizeof(float) * 7 * c->last_p));
    IRO_TRY(codec_alloc_t(c.get(), &c->head_b, sizeof(float)));
    IRO_TRY(codec_alloc_t(c.get(), &c->X, sizeof(float) * xe));
    IRO_TRY(codec_alloc(c.get(), &c->S, es * se));
    IRO_TRY(codec_alloc(c.get(), &c->S3, es * se));
    IRO_TRY(codec_alloc(c.get(), &c->S2, es * s2e));
    IRO_TRY(codec_alloc_t(c.get(), &c->lat, sizeof(float) * (size_t)g.max_frames * g.latent_dim));
    IRO_TRY(codec_alloc_t(c.get(), &c->wav, sizeof(float) * (size_t)g.max_frames * hop));
    *out = c.release();
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_codec_load_weights(irodori_codec* c, const irodori_codec_weights* w) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && w, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(w->out_proj_w && w->stem_w && w->blocks && w->head_alpha && w->head_w, IRODORI_ERR_INVALID_ARG,
                "null codec weight");
    const auto& g = c->cfg;
    for (int i = 0; i < g.num_blocks; i++) {
        const irodori_codec_block_weights& bw = w->blocks[i];
        IRO_REQUIRE(bw.alpha && bw.convt_w, IRODORI_ERR_INVALID_ARG, "null codec block weight");
        for (int u = 0; u < 3; u++)
            IRO_REQUIRE(bw.res_alpha0[u] && bw.res_conv_w[u] && bw.res_alpha1[u] && bw.res_pw_w[u],
                        IRODORI_ERR_INVALID_ARG, "null codec residual-unit weight");
    }
    IRO_HIP_CHECK(hipSetDevice(c->device));
    c->loaded = false;
    // out_proj: Burn [proj, latent, 1] is already [P, Cl] row-major.
    std::vector<float> inw((size_t)c->proj_p * g.latent_dim, 0.f);
    std::copy(w->out_proj_w, w->out_proj_w + (size_t)g.proj_dim * g.latent_dim, inw.begin());
    IRO_TRY(put_f32(c, c->in_w, inw));
    IRO_TRY(put_f32(c, c->in_b, padded(w->out_proj_b, g.proj_dim, c->proj_p)));
    const int slice = 128 / (int)c->esz;
    IRO_TRY(put_operand(c, c->stem_w, conv_rows(w->stem_w, g.decoder_dim, g.proj_dim, 7, c->dim_p, c->proj_p,
                                                round_to(7 * c->proj_p, slice))));
    if (w->stem_b) {
        if (!c->stem_b) IRO_TRY(codec_alloc_t(c, &c->stem_b, sizeof(float) * c->dim_p));
        IRO_TRY(put_f32(c, c->stem_b, padded(w->stem_b, g.decoder_dim, c->dim_p)));
    } else {
        c->stem_b = nullptr;
    }
    for (int i = 0; i < g.num_blocks; i++) {
        CodecBlock& b = c->blocks[i];
        const irodori_codec_block_weights& bw = w->blocks[i];
        IRO_TRY(put_f32(c, b.alpha, snake_consts(bw.alpha, b.cin, b.cin_p)));
        IRO_TRY(put_operand(c, b.wt, convt_rows(bw.convt_w, b.cin, b.cout, b.rate, b.cin_p, b.cout_p)));
        IRO_TRY(put_f32(c, b.bt, padded(bw.convt_b, b.cout, b.cout_p, b.rate)));
        for (int u = 0; u < 3; u++) {
            IRO_TRY(put_f32(c, b.ra0[u], snake_consts(bw.res_alpha0[u], b.cout, b.cout_p)));
            IRO_TRY(put_f32(c, b.ra1[u], snake_consts(bw.res_alpha1[u], b.cout, b.cout_p)));
            IRO_TRY(put_operand(c, b.rw[u], conv_rows(bw.res_conv_w[u], b.cout, b.cout, 7, b.cout_p, b.cout_p,
                                                      round_to(7 * b.cout_p, slice))));
            IRO_TRY(put_operand(c, b.pw[u], conv_rows(bw.res_pw_w[u], b.cout, b.cout, 1, b.cout_p, b.cout_p,
                                                      round_to(b.cout_p, slice))));
            if (bw.res_conv_b[u]) {
                if (!b.rb[u]) IRO_TRY(codec_alloc_t(c, &b.rb[u], sizeof(float) * b.cout_p));
                IRO_TRY(put_f32(c, b.rb[u], padded(bw.res_conv_b[u], b.cout, b.cout_p)));
            } else {
                b.rb[u] = nullptr;
            }
            if (bw.res_pw_b[u]) {
                if (!b.pb[u]) IRO_TRY(codec_alloc_t(c, &b.pb[u], sizeof(float) * b.cout_p));
                IRO_TRY(put_f32(c, b.pb[u], padded(bw.res_pw_b[u], b.cout, b.cout_p)));
            } else {
                b.pb[u] = nullptr;
            }
        }
    }
    const int Cl = g.decoder_dim >> g.num_blocks;
    IRO_TRY(put_f32(c, c->head_alpha, snake_consts(w->head_alpha, Cl, c->last_p)));
    std::vector<float> hw((size_t)7 * c->last_p, 0.f);
    for (int ch = 0; ch < Cl; ch++)
        for (int j = 0; j < 7; j++) hw[(size_t)j * c->last_p + ch] = w->head_w[(size_t)ch * 7 + j];
    IRO_TRY(put_f32(c, c->head_w, hw));
    IRO_TRY(put_f32(c, c->head_b, std::vector<float>{w->head_b ? w->head_b[0] : 0.f}));
    c->loaded = true;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_codec_hop_length(const irodori_codec* c) { return c ? c->hop : 0; }

int irodori_codec_decode_device(irodori_codec* c, int batch, int frames, const float* latent, float* wav,
                                void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && latent && wav, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(batch > 0 && frames > 0 && frames <= c->cfg.max_frames, IRODORI_ERR_SHAPE,
                "codec batch must be positive and frames in [1, max_frames]");
    IRO_REQUIRE(c->loaded, IRODORI_ERR_NOT_LOADED, "codec weights not loaded");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    return codec_decode(c, batch, frames, latent, wav, stream ? static_cast<hipStream_t>(stream) : c->stream);
    IRO_GUARD_END
}

int irodori_codec_decode(irodori_codec* c, int batch, int frames, const float* latent, float* wav) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && latent && wav, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(batch > 0 && frames > 0 && frames <= c->cfg.max_frames, IRODORI_ERR_SHAPE,
                "codec batch must be positive and frames in [1, max_frames]");
    IRO_REQUIRE(c->loaded, IRODORI_ERR_NOT_LOADED, "codec weights not loaded");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const size_t nl = (size_t)frames * c->cfg.latent_dim, nw = (size_t)frames * c->hop;
    for (int b = 0; b < batch; b++) {
        IRO_HIP_CHECK(hipMemcpyAsync(c->lat, latent + b * nl, sizeof(float) * nl, hipMemcpyHostToDevice, c->stream));
        IRO_TRY(codec_decode(c, 1, frames, c->lat, c->wav, c->stream));
        IRO_HIP_CHECK(hipMemcpyAsync(wav + b * nw, c->wav, sizeof(float) * nw, hipMemcpyDeviceToHost, c->stream));
        IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    }
    return IRODORI_OK;
    IRO_GUARD_END
}

}  // extern "C"
