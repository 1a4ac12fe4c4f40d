// Host-side launchers for the gfx950 kernels (one .hip file per kernel family).
// All launchers validate nothing themselves: callers (context.hip, the op entry points)
// check shapes against what each kernel's grid assumes before launching.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace irodori {

// Where the adaLN modulation vectors of a forward live: a table of rows
// [vec][layer][kind(attn,mlp)][chunk(shift,scale,gate)][D] (gate already tanh'd).
// Row index for batch row b: vec = (*step + step_add) * step_stride + (b / rows_per_vec).
struct ModTable {
    const float* tab;
    const int* step;   // device step counter (0 for single forwards)
    int step_stride;   // vectors per step
    int rows_per_vec;  // batch rows sharing one vector
    int layers;
    int step_add = 0;  // evaluation offset (1: the Heun corrector at t_{i+1})
    int vec_base = 0;  // first vector (a launch over one batch row of a multi-row table)
};
__host__ __device__ inline int mod_vec_index(const ModTable& mt, int step, int b) {
    return (step + mt.step_add) * mt.step_stride + b / mt.rows_per_vec + mt.vec_base;
}

// Position of latent/context key s inside a V^T row.  bf16 path (32x32x16 attention):
// bits 2 and 3 of the key index swapped; f32 path (16x16 attention): keys permuted inside
// each 32-key group.  Both are involutions on aligned groups, so padding stays in place.
__host__ __device__ inline int vt_pos_bf16(int s) { return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1); }
__host__ __device__ inline int vt_pos_f32(int s) {
    int kk = s & 31;
    return (s & ~31) | (((kk & 15) >> 2) * 8 + (kk >> 4) * 4 + (kk & 3));
}

// ---- kernels_norm.hip ------------------------------------------------------------------
void launch_rms_norm_op(const float* x, const float* w, int rows, int D, float eps, float* y,
                        hipStream_t st);
void launch_fused_adaln_op(const float* x, const float* scale, const float* shift, int B, int S,
                           int D, float eps, float* y, hipStream_t st);
// h = x / sqrt(mean(x^2)+eps) * (1 + scale) + shift for (layer, kind) of the table.
template <typename T>
void launch_norm_mod(const float* x, T* h, int M, int S, int D, float eps, ModTable mt,
                     int layer, int kind, hipStream_t st, uint8_t* q8 = nullptr,
                     uint8_t* q8s = nullptr);
// x[b] = x_src[b mod src_batches] @ in_w + in_b (in_proj), then h = norm_mod(x) for
// (layer 0, attn); b is the batch row.  h is nullable; q8 / q8s (nullable) receive the fp8
// GEMM-operand form of h (e4m3 codes, E8M0 scales per 32 values; D % 32 == 0).
// rstat (nullable; the fused adaLN of the bf16 model path, see GemmArgs): h gets
// x (1 + scale) and rstat [M, D/32] the row sums of x^2 per 32 columns instead.
// copies > 1: M rows computed, every output also written to the copies - 1 following
// M-row blocks (rows that share their source row and modulation vector).
template <typename T>
void launch_inproj_norm(const float* x_src, int src_batches, const float* in_w,
                        const float* in_b, float* x, T* h, int M, int S, int P, int D,
                        float eps, ModTable mt, hipStream_t st, uint8_t* q8 = nullptr,
                        uint8_t* q8s = nullptr, float* rstat = nullptr, int copies = 1);
// The fused adaLN operand of (layer, kind) from x: h = x (1 + scale), rstat [M, D/32].
template <typename T>
void launch_mod_stats(const float* x, T* h, int M, int S, int D, ModTable mt, int layer, int kind, float* rstat,
                      hipStream_t st);
// Shift rows of the modulation table as GEMM operands: stage[(l * 2 + k) * cap + v][D] =
// shift of (vector v, layer l, kind k) in bf16, for v < nvec.
void launch_shift_stage(const float* tab, int nvec, int cap, int L, int D, bf16* stage, hipStream_t st);


// One model evaluation of the RF sampler, as the update kernel applies it
// (euler_sampler.rs:435-714): the guided velocity v = v_0 + sum_k (v_0 - v_{role_k}) s_k
// over the role-major head outputs, the temporal score rescale v = (v omt + x) ratio / omt
// - x / omt (math.rs:38-53) at the evaluation's t when rescale != 0, then the integrator.
struct RfEval {
    float dt;          // t_{i+1} - t_i of the step
    float omt, ratio;  // 1 - t and the rescale ratio at the evaluation's t
    int rescale;
    int nterm;         // CFG terms
    int role[3];
    float scale[3];
    int ab_order;      // PLMS-4: history entries (newest first) after this step's push
};
enum RfMethod { RF_EULER = 0, RF_HEUN = 1, RF_PLMS4 = 2 };
// Evaluation (step, phase) of the plan is plan[2 * (*step) + phase]; phase 1 is the Heun
// corrector.  Euler: x += v dt.  Heun phase 0: hist = v, xin = x + v dt; phase 1:
// x += (hist + v) / 2 dt (the evaluation state is xin).  PLMS-4: hist slot (step mod 4) =
// v, x += sum of the Adams-Bashforth coefficients of order ab_order times the newest
// entries (euler_sampler.rs:98-117).
struct RfUpdateArgs {
    float* x;     // [n] sampler state
    float* xin;   // [n] Heun predictor state
    float* hist;  // [4][n]
    const RfEval* plan;  // null: no update (plain output head)
    int* step;
    int* done;    // advance set: workgroups finished, 0 between launches
    int advance;  // the last workgroup to finish sets done = 0 and *step += 1
    int phase, method;
    int n;        // U * S * P
};

// Element j of the state after the guided velocity v of evaluation e (f32, in the
// reference's operation order); x = a.x[j], loaded by the caller.
__device__ inline void rf_apply(const RfUpdateArgs& a, const RfEval& e, int step, int j, float v, float x) {
    const bool corr = a.method == RF_HEUN && a.phase == 1;
    const float xs = corr ? a.xin[j] : x;
    if (e.rescale) v = (v * e.omt + xs) * e.ratio / e.omt - xs / e.omt;  // math.rs:38-53
    if (a.method == RF_EULER) {
        a.x[j] = x + v * e.dt;
    } else if (a.method == RF_HEUN) {
        if (a.phase == 0) {
            a.hist[j] = v;
            a.xin[j] = x + v * e.dt;
        } else {
            a.x[j] = x + (a.hist[j] + v) / 2.0f * e.dt;
        }
    } else {
        const size_t n = (size_t)a.n;
        a.hist[(size_t)(step & 3) * n + j] = v;
        float ve = v;
        if (e.ab_order >= 2) {
            const float h1 = a.hist[(size_t)((step - 1) & 3) * n + j];
            if (e.ab_order == 2) {
                ve = v * 1.5f + h1 * -0.5f;
            } else {
                const float h2 = a.hist[(size_t)((step - 2) & 3) * n + j];
                if (e.ab_order == 3) {
                    ve = v * (23.0f / 12.0f) + h1 * (-16.0f / 12.0f) + h2 * (5.0f / 12.0f);
                } else {
                    const float h3 = a.hist[(size_t)((step - 3) & 3) * n + j];
                    ve = v * (55.0f / 24.0f) + h1 * (-59.0f / 24.0f) + h2 * (37.0f / 24.0f) + h3 * (-9.0f / 24.0f);
                }
            }
        }
        a.x[j] = x + ve * e.dt;
    }
}

// Output head: v[b,s,:] = out_proj(out_norm(x[b,s,:])) into v_out [B,S,P]; or, with
// rf.plan set, the sampler evaluation's head and update fused: for each of the B = U
// utterances, the rows role[k] * U + u of its nrole active roles (role[0] = 0, increasing),
// their velocities combined as v = v_0 + sum_k (v_0 - v_{role_k}) s_k per the plan, then
// rf_apply.
struct FinalArgs {
    const float* x;
    const float* norm_w;
    const float* out_w;   // [D, PT] = out_norm.weight (.) W_out, PT = 32, 64, 128 or 256 (the least >= P), zero past P
    const float* out_b;   // [P]
    int B, S, D, P;
    float eps;
    float* v_out;         // [B,S,P] (plain head)
    int nrole;            // sampler evaluation: active roles
    int role[3];
    RfUpdateArgs rf;
};
void launch_final(const FinalArgs& a, hipStream_t st);

// Speaker-KV scaling of cached context (kv_scaling.rs:10-60) on the device copies the
// attention reads: for rows < rows_scaled, the keys [aux_start, t_ctx) of K
// ([R, H, T1, Dh]) and V^T ([R, H, Dh, vs1], key order vt_pos_bf16 with bf16_order, else
// vt_pos_f32) times factor; src == dst scales in place, otherwise every other element is
// copied unchanged.  Dh a multiple of 8.
template <typename T>
void launch_scale_ctx_aux(const T* src_k, const T* src_v, T* dst_k, T* dst_v, int rows,
                          int rows_scaled, int H, int Dh, bool bf16_order, int T1, int vs1, int t_ctx,
                          int aux_start, float factor, hipStream_t st);
void launch_scale_copy(const float* src, float* dst, int n, float s, hipStream_t st);

// ---- kernels_ops.hip -------------------------------------------------------------------
// The joint-attention operator's staging: latent q, k, v [B, S, H, 64] f32 and gate logits
// [B, S, H*64] f32 (nullable: gate 1) into the layouts the QKV+gate epilogue writes -- Q
// [B, H, S, 64] head-normed (q_norm / k_norm [H, 64], nullable: no norm), half-RoPE'd
// (heads < H/2, tables [S, 32]) and pre-scaled by q_scale; K likewise without the scale;
// V^T [B, H, 64, vt_stride] at vt_pos_bf16 (T = bf16) / vt_pos_f32 (T = float), keys S ..
// vt_stride - 1 zero (vt_stride = S rounded up to 64); G = sigmoid(gate).
template <typename T>
void launch_attn_op_stage(const float* q, const float* k, const float* v, const float* gate, const float* q_norm,
                          const float* k_norm, const float* rope_cos, const float* rope_sin, int B, int S, int H,
                          float eps, float q_scale, int vt_stride, T* Q, T* K, T* Vt, T* G, hipStream_t st);
template <typename T>
void launch_to_f32(const T* src, long n, float* dst, hipStream_t st);
// Modulation vectors [B, D] (shift, scale, gate as applied) into table rows vec b, (layer,
// kind) of tab [vec][layer][2][3][D].
void launch_put_mod_vectors(const float* shift, const float* scale, const float* gate, int B, int D, int layers,
                            int layer, int kind, float* tab, hipStream_t st);

// ---- kernels_cond.hip ------------------------------------------------------------------
struct VecLinJob {
    const float* X;  // [nvec, ldx]
    const float* W;  // [K, N] row-major
    const float* bias;  // [N] or null
    const float* R;  // residual [nvec, ldr] or null
    float* Y;        // [nvec, ldy]
    int ldx, ldr, ldy, K, N;
    int act_in;   // 0 none, 1 silu
    int act_out;  // 0 none, 1 silu, 2 tanh
};
void launch_timestep_embedding(const float* t, int nvec, int t_dim, float* out, hipStream_t st);
void launch_vec_linear(const VecLinJob* d_jobs, int njobs, int nvec, int max_n, hipStream_t st);

// ---- kernels_gemm.hip ------------------------------------------------------------------
enum GemmEpi {
    EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKVG = 3, EPI_CTXKV = 4, EPI_ADD = 5, EPI_SNAKE = 6, EPI_RESUNIT = 7
};
template <typename T>
struct GemmArgs {
    const T* A;   // [M, K] row-major
    const T* W;   // [N, K] row-major (K contiguous), or tile-major with w_tiled
    int M, N, K;
    // w_tiled: W (and W8) stored tile-major, as launch_tile_rows writes it: each group of 64
    // rows holds its K * element-size / 128 slices one after the other, a slice being the
    // group's 64 rows x 128 bytes (8 KB contiguous).  A group spans the same bytes as in the
    // row-major layout.  Not for convolutions; BN a multiple of 64.
    int w_tiled;
    // EPI_STORE: C [M, N] f32
    float* C;
    // EPI_RESID: x[m, n] += gate[vec(b), n] * acc, b = m / S
    float* x;
    ModTable mt;
    int layer, kind;
    int S;
    // EPI_SWIGLU: U [M, N/2] = silu(acc_1) * acc_3 (W rows interleaved in 32-row groups)
    T* U;
    // EPI_QKVG: N = 4 * D; q/k head-normed (+ half RoPE), v raw, gate sigmoid.
    T* Q;  // [B, H, S, Dh]
    T* Kd; // [B, H, S, Dh]
    T* Vd; // V^T [B, H, Dh, vt_stride], key s at vt_pos_bf16 / vt_pos_f32 by dtype
    int vt_stride;  // multiple of 64, >= S
    float q_scale;  // q multiplier (Dh^-1/2 * log2 e) applied after norm + RoPE
    T* G;  // [M, D]
    const float* q_norm;  // [H, Dh]
    const float* k_norm;
    const float* rope_cos;  // [S, Dh/2]
    const float* rope_sin;
    const float* rope_cs;   // [S, Dh/2, 2]: the same (cos, sin) pairs interleaved
    int H, D;
    float eps;
    // EPI_CTXKV (context KV build, attention.rs:431-501): N = 2 H Dh columns [K | V] of the
    // context rows key_off .. key_off + M - 1: K head-normed with k_norm into Ck
    // [H, ctx_stride, Dh], V into Cv = V^T [H, Dh, ctx_vstride] at vt_pos_bf16 / vt_pos_f32.
    T* Ck;
    T* Cv;
    int key_off, ctx_stride, ctx_vstride;
    // EPI_ADD: x[m, n] = (x[m, n] + acc) * rmask[m] (rmask nullable: 1), the encoder's
    // plain residual with its per-block re-masking (text_encoder.rs:131-145).
    const float* rmask;
    // fp8 operands (launch_gemm_fp8): A8 [M, K] e4m3 with As [M, K/32] E8M0 block scales
    // (power-of-two scale of row m, k block kb = 2^(As - 127)); W8 [N, K] e4m3 with f32
    // per-output-channel scales ws [N].  C = (A8 * 2^As) @ W8^T * ws.
    const uint8_t* A8;
    const uint8_t* As;
    const uint8_t* W8;
    const float* ws;
    // EPI_SWIGLU over fp8 operands: U in the fp8 GEMM-operand form (e4m3 codes U8 [M, N/2],
    // E8M0 scales U8s [M, N/64]) for the next projection, instead of U.
    uint8_t* U8;
    uint8_t* U8s;
    // Convolution epilogues (the codec decoder): EPI_STORE and EPI_ADD add bias[n] when it
    // is set; EPI_SNAKE writes U [M, N] = Snake(acc + bias[n]) in the operand dtype,
    // Snake(v, a) = v + sin(a v)^2 / (a + 1e-9) (codec/layers.rs:24-31), alpha the block
    // [3, alpha_n] = (a, a / pi, 0.5 / (a + 1e-9)) of channel n % alpha_n (bf16: hardware
    // cosine, f32: sinf).  EPI_STORE / EPI_ADD with U set also write U[i] = Snake(out[i])
    // for the linear indices i = row * N + n in [u_lo, u_hi): the next convolution's
    // operand, produced without another pass over the result.
    const float* bias;
    const float* alpha;
    int alpha_n;
    long u_lo, u_hi;
    // EPI_RESUNIT (launch_gemm_conv, one tile column: N = 64, 96, 128 or 192): the codec
    // ResidualUnit's tail after its dilated conv, x[M, N] += Snake(acc + bias) @ W2^T +
    // bias2 (W2 [N, K2] with K2 = N rounded up to 64 / 32 columns for bf16 / f32, zero
    // past N: the 1x1 conv; Snake with alpha), then U = Snake(x) with alpha2 when U is set.
    // The Snake'd tile never leaves LDS.
    const T* W2;
    const float* bias2;
    const float* alpha2;
    // launch_gemm_conv: A is an implicit im2col.  Row m of the GEMM, k = j * conv_cp + c
    // reads A[(m + j * conv_dil) * conv_cp + c] (A points at the source row the first tap
    // of output row 0 reads); source rows at or past conv_rows read as zero.  conv_cp is a
    // multiple of half a 128-byte slice; K spans the taps rounded up to whole slices (the
    // weights are zero there).
    int conv_cp, conv_dil, conv_rows;
    // Fused adaLN of the model path (bf16 operands, norm.rs:160-169): with r =
    // rsqrt(mean(x^2) + eps), h = x r (1 + scale) + shift, so h W = r (x (1 + scale)) W + shift W.
    //   consumer (EPI_QKVG / EPI_SWIGLU with rstat set): A holds x (1 + scale) and rstat
    //   [M, K/32] the sums of x^2 per 32 columns; each accumulator row is multiplied by r
    //   and rbias[vec, n] (= shift W of the launch's one modulation vector, [nvec, N]) is
    //   added before the epilogue.  Every row must map to the same vector (a sampler
    //   evaluation, where all rows share the step's t).
    //   producer (EPI_RESID with Hn set): after x += gate * acc, writes Hn [M, N] =
    //   x (1 + scale of (next_layer, next_kind)) and rstat_out [M, N/32].
    const float* rstat;
    const float* rbias;
    T* Hn;
    float* rstat_out;
    int next_layer, next_kind;
};
template <typename T>
int launch_gemm(int epi, const GemmArgs<T>& a, hipStream_t st);
// The same epilogues over fp8 operands (K % 128 == 0); outputs in bf16 / f32 as above.
int launch_gemm_fp8(int epi, const GemmArgs<bf16>& a, hipStream_t st);
// Row-major [N, row_bytes] -> the tile-major weight layout of GemmArgs::w_tiled (N a
// multiple of 64, row_bytes of 128).  A weight slice of a 128- or 64-wide tile is then one or
// two 8 KB runs instead of 64 or 128 rows of 128 bytes a row apart, so a tile's weight
// loads open far fewer DRAM pages.
void launch_tile_rows(const void* src, int N, int row_bytes, void* dst, hipStream_t st);
// Convolution as a GEMM over an implicit im2col (conv_* fields): K = taps * conv_cp rounded
// up to whole 128-byte slices, conv_cp a multiple of half a slice; EPI_STORE, EPI_ADD,
// EPI_SNAKE or EPI_RESUNIT.
template <typename T>
int launch_gemm_conv(int epi, const GemmArgs<T>& a, hipStream_t st);

// ---- kernels_enc.hip -------------------------------------------------------------------
// Host f32 [K, N] (Burn layout, on the device) -> K-major [N, K]; mode 1 interleaves the
// W1 / W3 halves per 32 rows (the SwiGLU GEMM's layout).
template <typename T>
void launch_transpose(const float* src, int K, int N, int mode, T* dst, hipStream_t st);
void launch_enc_embed(const int* ids, const float* emb, const float* mask, float* x, int M, int E, hipStream_t st);
void launch_enc_inproj(const float* lat, const float* w, const float* b, const float* mask, float* x, int M, int K,
                       int E, hipStream_t st);
template <typename TO>
void launch_rmsnorm_w(const float* x, const float* w, int M, int E, float eps, TO* y, int ystride, hipStream_t st);
template <typename T>
void launch_enc_head_prep(const float* qkvg, const float* q_norm, const float* k_norm, const float* cs, const float* sn,
                          int M, int S, int H, int Dh, float eps, T* q, T* k, T* v, T* gate, hipStream_t st);
void launch_enc_mean_token(float* out, const float* mask, uint8_t* mask_out, int B, int S, int E, hipStream_t st);

// ---- kernels_codec.hip -----------------------------------------------------------------
// DACVAE decoder operands: channels-last [frames, Cp] (Cp % 8 == 0), convolution operands
// with `halo` zero rows on both sides of the L frames ([L + 2 halo, Cp]).  A Snake's
// `alpha` is the block [3, Cp] = (a, a / pi, 0.5 / (a + 1e-9)); T = bf16 evaluates it with
// the hardware cosine, T = float with sinf.
template <typename T>
void launch_codec_in(const float* lat, int frames, int Cl, const float* w, const float* b, int Pp, int halo, T* s,
                     hipStream_t st);
// WmHead with its Snake over x [L, Cp] f32 (Cp a multiple of 64, at most 256).
template <typename T>
void launch_codec_head(const float* x, int L, int Cp, const float* alpha, const float* w, const float* b, float* wav,
                       hipStream_t st);
template <typename T>
void launch_cvt_f32(const float* src, long n, T* dst, hipStream_t st);
template <typename T>
void launch_codec_zero_halo(T* s, int L, int Cp, int halo, hipStream_t st);

// ---- kernels_fp8.hip -------------------------------------------------------------------
// Weights w [N, K] f32 (K-major, K % 4 == 0) -> e4m3 codes q [N, K], channel scales s [N].
void launch_quant_weight_rows(const float* w, int N, int K, uint8_t* q, float* s, hipStream_t st);
// Activations x [M, K] (K % 32 == 0) -> e4m3 codes q [M, K], E8M0 block scales s [M, K/32].
template <typename T>
void launch_mx_quant_rows(const T* x, int M, int K, uint8_t* q, uint8_t* s, hipStream_t st);

// ---- kernels_attn.hip ------------------------------------------------------------------
template <typename T>
struct AttnArgs {
    const T* Q;        // [B, H, Sq, Dh]
    // segment 0 (latent self keys): [B, H, seg0_stride, Dh], len0 keys, no mask
    const T* K0;
    const T* V0;
    int len0, stride0;
    const float* mask0;  // optional [B, len0]; value < 0.5 = masked out
    // optional [B, ceil(len0/64)]: bit k of tile t set iff latent key 64 t + k attends
    // (launch_attention32; required there together with mask0)
    const unsigned long long* bits0;
    // segment 1 (cached context keys): [B, H, stride1, Dh], len1 keys
    const T* K1;
    const T* V1;
    int len1, stride1;
    const float* mask1;   // optional [B, stride1]; value < 0.5 = masked out
    const int* tile_on1;  // [B, ceil(stride1/64)] nonzero if the 64-key tile has a valid key
    // [B, ceil(stride1/64)]: bit k of tile t set iff key 64 t + k is valid (launch_attention32)
    const unsigned long long* bits1;
    int B, H, Sq;
    float scale;
    // v_transposed: V0/V1 hold V^T [B, H, Dh, vstride] with keys at vt_pos_f32 (this
    // kernel) or vt_pos_bf16 (launch_attention32); vstride is a multiple of 64 and padding
    // columns hold finite values.
    bool v_transposed;
    int vstride0, vstride1;
    // prescaled: Q already multiplied by scale * log2(e) (the QKV epilogue does this).
    bool prescaled;
    // epilogue: out_mode 0 -> O [B*Sq, H*Dh] (T) = gate[m, h*Dh+d] * attn;
    //           out_mode 1 -> Of [B, H, Sq, Dh] f32;
    //           out_mode 2 -> the out_mode 0 values in the fp8 GEMM-operand form: e4m3
    //           codes O8 [B*Sq, H*Dh] and E8M0 scales O8s [B*Sq, H*Dh/32] (bf16 kernel only)
    int out_mode;
    const T* G;
    T* O;
    float* Of;
    uint8_t* O8;
    uint8_t* O8s;
};
template <typename T, int DH>
int launch_attention(const AttnArgs<T>& a, hipStream_t st);
// bf16 / f16, Dh = 64, V^T in vt_pos_bf16 order, Q pre-scaled (kernels_attn32.hip).  The
// latent and context segments together hold at most kAttnMaxKeyTiles 64-key tiles.
constexpr int kAttnMaxKeyTiles = 256;
int launch_attention32(const AttnArgs<bf16>& a, hipStream_t st);
int launch_attention32(const AttnArgs<f16>& a, hipStream_t st);
// The SDPA operator on 16-bit operands with Dh = 64 through attn32_kernel: q, k, v
// [B, H, S, 64] as given, mask [B, Skv] f32 (>= 0.5 attends; nullable), out [B, H, Sq, 64]
// f32.  Q (pre-scaled), V^T and the key bits are staged in ws (256-byte aligned, at least
// sdpa_stage_bytes); Skv <= 64 * kAttnMaxKeyTiles.  Returns -1 on a shape the kernel does not take.
size_t sdpa_stage_bytes(int B, int H, int Sq, int Skv);
template <typename T>
int launch_sdpa_staged(const T* q, const T* k, const T* v, const float* mask, int B, int H, int Sq, int Skv,
                       float scale, float* out, void* ws, size_t ws_bytes, hipStream_t st);

}  // namespace irodori
