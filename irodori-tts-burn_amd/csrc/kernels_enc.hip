// Weight ingest and the condition-encoder kernels (TextEncoder / ReferenceLatentEncoder,
// text_encoder.rs:17-148, speaker_encoder.rs:85-162, attention.rs:52-127): the front ends
// (token embedding, latent in_proj / 6), RMSNorm with weight, the per-head q / k norm with
// full RoPE, and the speaker conditioner's masked-mean token.  The encoder's projections
// run on the GEMM kernel and its attention on the generic flash-attention kernel.
#include "common.hpp"
#include "kernels.hpp"

namespace irodori {

namespace {

// ---------------------------------------------------------------------------------------
// Weight ingest: Burn [K, N] f32 -> K-major [N, K] compute dtype.
// mode 0: dst row n = source column n.
// mode 1: SwiGLU interleave — dst rows 64g..64g+31 = W1 columns 32g.., rows 64g+32..64g+63 =
//         W3 columns 32g.. (W3 starts at source column N/2).
// ---------------------------------------------------------------------------------------
template <typename T>
__global__ void transpose_kmajor_kernel(const float* __restrict__ src, int K, int N, int mode,
                                        T* __restrict__ dst) {
    __shared__ float tile[32][33];
    int k0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
    int tx = threadIdx.x, ty = threadIdx.y;  // 32 x 8
    for (int r = ty; r < 32; r += 8) {
        int k = k0 + r, n = n0 + tx;
        int sc = n;
        if (mode == 1 && n < N) {
            int half = N / 2, g = n / 64, w = n % 64;
            sc = w < 32 ? 32 * g + w : half + 32 * g + (w - 32);
        }
        tile[r][tx] = (k < K && n < N) ? src[(size_t)k * N + sc] : 0.f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        int n = n0 + r, k = k0 + tx;
        if (n < N && k < K) dst[(size_t)n * K + k] = from_f32<T>(tile[tx][r]);
    }
}

// x[m] = embedding[ids[m]] * mask[m] (TextEncoder::forward, text_encoder.rs:121-129).
__global__ __launch_bounds__(256) void enc_embed_kernel(const int* __restrict__ ids, const float* __restrict__ emb,
                                                        const float* __restrict__ mask, float* __restrict__ x, int E) {
    const int m = blockIdx.x;
    const float mk = mask[m];
    const float* er = emb + (size_t)ids[m] * E;
    for (int d = threadIdx.x; d < E; d += 256) x[(size_t)m * E + d] = mk != 0.f ? er[d] : 0.f;
}

// x[m] = (latent[m] @ in_w + in_b) / 6 * mask[m] (ReferenceLatentEncoder::forward,
// speaker_encoder.rs:140-148); one block per row, threads over the output columns.
__global__ __launch_bounds__(256) void enc_inproj_kernel(const float* __restrict__ lat, const float* __restrict__ w,
                                                         const float* __restrict__ bias, const float* __restrict__ mask,
                                                         float* __restrict__ x, int K, int E) {
    extern __shared__ float lrow[];
    const int m = blockIdx.x;
    for (int k = threadIdx.x; k < K; k += 256) lrow[k] = lat[(size_t)m * K + k];
    __syncthreads();
    const float mk = mask[m];
    for (int d = threadIdx.x; d < E; d += 256) {
        float acc = bias[d];
        for (int k = 0; k < K; k++) acc += lrow[k] * w[(size_t)k * E + d];
        x[(size_t)m * E + d] = mk != 0.f ? acc / 6.f : 0.f;
    }
}

// y[m] = x[m] / sqrt(mean(x[m]^2) + eps) * w (RmsNorm::forward, norm.rs:25-39); one
// wavefront per row.
template <typename TO>
__global__ __launch_bounds__(256) void rmsnorm_w_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        int M, int E, float eps, TO* __restrict__ y, int ystride) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (m >= M) return;
    const float* xr = x + (size_t)m * E;
    float ss = 0.f;
    for (int d = lane; d < E; d += 64) ss += xr[d] * xr[d];
    ss = wave_sum(ss);
    const float rms = sqrtf(ss / (float)E + eps);
    for (int d = lane; d < E; d += 64) y[(size_t)m * ystride + d] = from_f32<TO>(xr[d] / rms * w[d]);
}

// From the projection [q | k | v | g] (f32 [M, 4E]): q and k head-RMSNormed (norm.rs:60-74)
// and rotated on every head (full RoPE, interleaved pairs, rope.rs:82-113) into
// [B, H, S, Dh]; v copied into [B, H, S, Dh]; gate = sigmoid(g) (attention.rs:117-120).
// One wavefront per (token, head); lane l owns dims 2l, 2l + 1 (Dh <= 128).
template <typename T>
__global__ __launch_bounds__(256) void enc_head_prep_kernel(const float* __restrict__ qkvg, const float* __restrict__ q_norm,
                                                            const float* __restrict__ k_norm, const float* __restrict__ cs,
                                                            const float* __restrict__ sn, int M, int S, int H, int Dh,
                                                            float eps, T* __restrict__ q, T* __restrict__ k,
                                                            T* __restrict__ v, T* __restrict__ gate) {
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (item >= M * H) return;
    const int m = item / H, h = item % H, b = m / S, s = m % S;
    const int E = H * Dh;
    const bool act = 2 * lane < Dh;
    const int d = 2 * lane;
    const float* row = qkvg + (size_t)m * 4 * E;
    const size_t o = (((size_t)b * H + h) * S + s) * Dh + d;
    const float c = act ? cs[(size_t)s * (Dh / 2) + lane] : 0.f, sv = act ? sn[(size_t)s * (Dh / 2) + lane] : 0.f;
#pragma unroll
    for (int which = 0; which < 2; which++) {  // q, k
        const float* src = row + which * E + h * Dh;
        const float a0 = act ? src[d] : 0.f, a1 = act ? src[d + 1] : 0.f;
        const float ss = wave_sum(a0 * a0 + a1 * a1);
        const float inv = 1.f / sqrtf(ss / (float)Dh + eps);
        const float* nw = (which ? k_norm : q_norm) + h * Dh;
        if (!act) continue;
        const float x0 = a0 * inv * nw[d], x1 = a1 * inv * nw[d + 1];
        T* dst = which ? k : q;
        dst[o] = from_f32<T>(x0 * c - x1 * sv);
        dst[o + 1] = from_f32<T>(x0 * sv + x1 * c);
    }
    if (act) {
        const float* vs = row + 2 * E + h * Dh;
        v[o] = from_f32<T>(vs[d]);
        v[o + 1] = from_f32<T>(vs[d + 1]);
        const float* gs = row + 3 * E + h * Dh;
        gate[(size_t)m * E + h * Dh + d] = from_f32<T>(1.f / (1.f + __expf(-gs[d])));
        gate[(size_t)m * E + h * Dh + d + 1] = from_f32<T>(1.f / (1.f + __expf(-gs[d + 1])));
    }
}

// The speaker conditioner's masked-mean token (prepend_masked_mean_token,
// aux_conditioner.rs:150-185): out[b, 0, :] = sum over valid s of out[b, 1 + s, :] /
// max(count, 1); mask_out[b, 0] = count > 0.  One block per (batch row, 256 columns).
__global__ __launch_bounds__(256) void enc_mean_token_kernel(float* __restrict__ out, const float* __restrict__ mask,
                                                             uint8_t* __restrict__ mask_out, int S, int E) {
    const int b = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
    float cnt = 0.f;
    for (int s = 0; s < S; s++) cnt += mask[(size_t)b * S + s] != 0.f ? 1.f : 0.f;
    if (d < E) {
        float acc = 0.f;
        float* ob = out + (size_t)b * (S + 1) * E;
        for (int s = 0; s < S; s++)
            if (mask[(size_t)b * S + s] != 0.f) acc += ob[(size_t)(1 + s) * E + d];
        ob[d] = acc / fmaxf(cnt, 1.f);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) mask_out[(size_t)b * (S + 1)] = cnt > 0.f ? 1 : 0;
}

}  // namespace

template <typename T>
void launch_transpose(const float* src, int K, int N, int mode, T* dst, hipStream_t st) {
    dim3 grid((K + 31) / 32, (N + 31) / 32), block(32, 8);
    transpose_kmajor_kernel<T><<<grid, block, 0, st>>>(src, K, N, mode, dst);
}
template void launch_transpose<float>(const float*, int, int, int, float*, hipStream_t);
template void launch_transpose<bf16>(const float*, int, int, int, bf16*, hipStream_t);

void launch_enc_embed(const int* ids, const float* emb, const float* mask, float* x, int M, int E, hipStream_t st) {
    enc_embed_kernel<<<M, 256, 0, st>>>(ids, emb, mask, x, E);
}

void launch_enc_inproj(const float* lat, const float* w, const float* b, const float* mask, float* x, int M, int K,
                       int E, hipStream_t st) {
    enc_inproj_kernel<<<M, 256, sizeof(float) * K, st>>>(lat, w, b, mask, x, K, E);
}

template <typename TO>
void launch_rmsnorm_w(const float* x, const float* w, int M, int E, float eps, TO* y, int ystride, hipStream_t st) {
    rmsnorm_w_kernel<TO><<<(M + 3) / 4, 256, 0, st>>>(x, w, M, E, eps, y, ystride);
}
template void launch_rmsnorm_w<float>(const float*, const float*, int, int, float, float*, int, hipStream_t);
template void launch_rmsnorm_w<bf16>(const float*, const float*, int, int, float, bf16*, int, hipStream_t);

template <typename T>
void launch_enc_head_prep(const float* qkvg, const float* q_norm, const float* k_norm, const float* cs, const float* sn,
                          int M, int S, int H, int Dh, float eps, T* q, T* k, T* v, T* gate, hipStream_t st) {
    enc_head_prep_kernel<T><<<(M * H + 3) / 4, 256, 0, st>>>(qkvg, q_norm, k_norm, cs, sn, M, S, H, Dh, eps, q, k, v, gate);
}
template void launch_enc_head_prep<float>(const float*, const float*, const float*, const float*, const float*, int, int,
                                          int, int, float, float*, float*, float*, float*, hipStream_t);
template void launch_enc_head_prep<bf16>(const float*, const float*, const float*, const float*, const float*, int, int,
                                         int, int, float, bf16*, bf16*, bf16*, bf16*, hipStream_t);

void launch_enc_mean_token(float* out, const float* mask, uint8_t* mask_out, int B, int S, int E, hipStream_t st) {
    enc_mean_token_kernel<<<dim3((E + 255) / 256, B), 256, 0, st>>>(out, mask, mask_out, S, E);
}

}  // namespace irodori
