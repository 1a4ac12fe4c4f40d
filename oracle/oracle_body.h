/*
 * Body of the CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Included twice by oracle.c with R = float / double and P(name) = orc_f32_name /
 * orc_f64_name.  Each function cites the reference lines whose semantics it restates.
 */

/* rope.rs:141-165 — emb = [cos(t*f_i) | sin(t*f_i)], f_i = 1000*exp(-ln(1e4)*i/half).
 * The reference computes the frequencies in f32; the f64 variant computes them in f64. */
void P(timestep_embedding)(const float* t, int B, int t_dim, float* out) {
    int half = t_dim / 2;
    R log_10000 = LOG(R_C(10000.0));
    for (int b = 0; b < B; b++) {
        for (int i = 0; i < half; i++) {
            R f = R_C(1000.0) * EXP((-log_10000 * (R)i) / (R)half);
            R a = (R)t[b] * f;
            out[b * t_dim + i] = (float)COS(a);
            out[b * t_dim + half + i] = (float)SIN(a);
        }
    }
}

/* rope.rs:24-63 — cos/sin tables [S, Dh/2], freq_i = 1/theta^(2i/Dh), angle = pos*freq_i. */
void P(rope_tables)(int S, int Dh, float theta, float* cos_out, float* sin_out) {
    int half = Dh / 2;
    for (int s = 0; s < S; s++) {
        for (int i = 0; i < half; i++) {
            R freq = R_C(1.0) / POW((R)theta, R_C(2.0) * (R)i / (R)Dh);
            R a = (R)s * freq;
            cos_out[s * half + i] = (float)COS(a);
            sin_out[s * half + i] = (float)SIN(a);
        }
    }
}

/* Burn Linear::forward in row layout: y[M,N] = x[M,K] @ w[K,N] (+ b[N]).
 * Blocked over rows and columns so each weight row streamed from cache serves
 * ORC_IB output rows. */
#define ORC_IB 16
#define ORC_JB 128
void P(linear)(const float* x, const float* w, const float* b, int M, int K, int N, float* y) {
    int nib = (M + ORC_IB - 1) / ORC_IB, njb = (N + ORC_JB - 1) / ORC_JB;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int blk = 0; blk < nib * njb; blk++) {
        int i0 = (blk / njb) * ORC_IB, j0 = (blk % njb) * ORC_JB;
        int ni = M - i0 < ORC_IB ? M - i0 : ORC_IB;
        int nj = N - j0 < ORC_JB ? N - j0 : ORC_JB;
        R acc[ORC_IB][ORC_JB];
        for (int r = 0; r < ni; r++)
            for (int j = 0; j < nj; j++) acc[r][j] = b ? (R)b[j0 + j] : R_C(0.0);
        for (int k = 0; k < K; k++) {
            const float* wr = w + (size_t)k * N + j0;
            for (int r = 0; r < ni; r++) {
                R a = (R)x[(size_t)(i0 + r) * K + k];
                R* ar = acc[r];
                for (int j = 0; j < nj; j++) ar[j] += a * (R)wr[j];
            }
        }
        for (int r = 0; r < ni; r++)
            for (int j = 0; j < nj; j++) y[(size_t)(i0 + r) * N + j0 + j] = (float)acc[r][j];
    }
}

/* norm.rs:25-39 (RmsNorm::forward) and rms_norm.rs:161-175 (reference_rms_norm):
 * y = x / sqrt(mean(x^2) + eps) * w. */
void P(rms_norm)(const float* x, const float* w, int rows, int D, float eps, float* y) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < rows; i++) {
        const float* xr = x + (size_t)i * D;
        R ss = 0;
        for (int d = 0; d < D; d++) ss += (R)xr[d] * (R)xr[d];
        R rms = SQRT(ss / (R)D + (R)eps);
        for (int d = 0; d < D; d++) y[(size_t)i * D + d] = (float)((R)xr[d] / rms * (R)w[d]);
    }
}

/* norm.rs:160-169 and fused_adaln.rs:223-251 (reference_fused_adaln):
 * y = x / sqrt(mean(x^2)+eps) * (1 + scale[b]) + shift[b]; no learnable norm weight. */
void P(fused_adaln)(const float* x, const float* scale, const float* shift, int B, int S, int D,
                    float eps, float* y) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < B * S; i++) {
        int b = i / S;
        const float* xr = x + (size_t)i * D;
        R ss = 0;
        for (int d = 0; d < D; d++) ss += (R)xr[d] * (R)xr[d];
        R rms = SQRT(ss / (R)D + (R)eps);
        for (int d = 0; d < D; d++)
            y[(size_t)i * D + d] =
                (float)((R)xr[d] / rms * (R_C(1.0) + (R)scale[b * D + d]) + (R)shift[b * D + d]);
    }
}

/* norm.rs:60-74 (HeadRmsNorm::forward): per (token, head) over Dh, times w[h, :]. */
void P(head_rms_norm)(const float* x, const float* w, int N, int H, int Dh, float eps, float* y) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < N * H; i++) {
        int h = i % H;
        const float* xr = x + (size_t)i * Dh;
        R ss = 0;
        for (int d = 0; d < Dh; d++) ss += (R)xr[d] * (R)xr[d];
        R rms = SQRT(ss / (R)Dh + (R)eps);
        for (int d = 0; d < Dh; d++)
            y[(size_t)i * Dh + d] = (float)((R)xr[d] / rms * (R)w[h * Dh + d]);
    }
}

/* rope.rs:82-113 (apply_rotary_emb) restricted to heads [h_lo, h_hi): interleaved pairs
 * (x[2k], x[2k+1]) rotated as a complex product by (cos[s,k], sin[s,k]). */
static void P(rope_heads)(const float* x, const float* cos_t, const float* sin_t, int B, int S,
                          int H, int Dh, int h_hi, float* y) {
    int half = Dh / 2;
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < B * S; i++) {
        int s = i % S;
        for (int h = 0; h < H; h++) {
            const float* xr = x + ((size_t)i * H + h) * Dh;
            float* yr = y + ((size_t)i * H + h) * Dh;
            if (h >= h_hi) {
                for (int d = 0; d < Dh; d++) yr[d] = xr[d];
                continue;
            }
            for (int k = 0; k < half; k++) {
                R c = (R)cos_t[s * half + k], sn = (R)sin_t[s * half + k];
                R re = (R)xr[2 * k], im = (R)xr[2 * k + 1];
                yr[2 * k] = (float)(re * c - im * sn);
                yr[2 * k + 1] = (float)(re * sn + im * c);
            }
        }
    }
}

/* rope.rs:119-135 (apply_rotary_half): RoPE on heads [0, H/2), heads [H/2, H) pass through. */
void P(rope_half)(const float* x, const float* cos_t, const float* sin_t, int B, int S, int H,
                  int Dh, float* y) {
    P(rope_heads)(x, cos_t, sin_t, B, S, H, Dh, H / 2, y);
}

/* rope.rs:82-113 on all heads (SelfAttention's full RoPE; used to pin the half variant). */
void P(rope_full)(const float* x, const float* cos_t, const float* sin_t, int B, int S, int H,
                  int Dh, float* y) {
    P(rope_heads)(x, cos_t, sin_t, B, S, H, Dh, H, y);
}

/* softmax(q k^T * scale + mask) v over [B, H, S, Dh] tensors; mask [B, Skv] with
 * value < 0.5 meaning masked-out, and a fully masked row yields exactly 0.
 * Follows reference_sdpa (fused_sdpa_native.rs:329-388) and the all-masked => 0 contract
 * of manual_sdpa (attention.rs:686-716, test attention.rs:770-787). */
void P(sdpa)(const float* q, const float* k, const float* v, const float* mask, int B, int H,
             int Sq, int Skv, int Dh, float scale, float* out) {
    #pragma omp parallel
    {
        R* sc = (R*)malloc(sizeof(R) * (size_t)(Skv > 0 ? Skv : 1));
        R* acc = (R*)malloc(sizeof(R) * (size_t)Dh);
        #pragma omp for schedule(static)
        for (int i = 0; i < B * H * Sq; i++) {
            int b = i / (H * Sq), bh = i / Sq;
            const float* qr = q + (size_t)i * Dh;
            R mx = -INFINITY;
            for (int j = 0; j < Skv; j++) {
                if (mask && mask[(size_t)b * Skv + j] < 0.5f) { sc[j] = -INFINITY; continue; }
                const float* kr = k + ((size_t)bh * Skv + j) * Dh;
                R dot = 0;
                for (int d = 0; d < Dh; d++) dot += (R)qr[d] * (R)kr[d];
                sc[j] = dot * (R)scale;
                if (sc[j] > mx) mx = sc[j];
            }
            R sum = 0;
            for (int d = 0; d < Dh; d++) acc[d] = 0;
            if (mx != -INFINITY) {
                for (int j = 0; j < Skv; j++) {
                    if (sc[j] == -INFINITY) continue;
                    R e = EXP(sc[j] - mx);
                    sum += e;
                    const float* vr = v + ((size_t)bh * Skv + j) * Dh;
                    for (int d = 0; d < Dh; d++) acc[d] += e * (R)vr[d];
                }
            }
            float* o = out + (size_t)i * Dh;
            for (int d = 0; d < Dh; d++) o[d] = sum > 0 ? (float)(acc[d] / sum) : 0.0f;
        }
        free(sc);
        free(acc);
    }
}

static R P(silu)(R v) { return v / (R_C(1.0) + EXP(-v)); }
static R P(sigmoid)(R v) { return R_C(1.0) / (R_C(1.0) + EXP(-v)); }

/* dit/model.rs:80-85 (CondModule::forward) after get_timestep_embedding (rope.rs:141-165):
 * c = L2(silu(L1(silu(L0(emb))))), no biases.  cond_out: [B, 3D]. */
void P(cond_module)(const orc_cfg* c, const orc_io* io, const float* t, int B, float* cond_out) {
    int D = c->model_dim, td = c->t_dim;
    float* emb = (float*)malloc(sizeof(float) * (size_t)B * td);
    float* h0 = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* h1 = (float*)malloc(sizeof(float) * (size_t)B * D);
    P(timestep_embedding)(t, B, td, emb);
    P(linear)(emb, io->cond_w0, NULL, B, td, D, h0);
    for (int i = 0; i < B * D; i++) h0[i] = (float)P(silu)((R)h0[i]);
    P(linear)(h0, io->cond_w1, NULL, B, D, D, h1);
    for (int i = 0; i < B * D; i++) h1[i] = (float)P(silu)((R)h1[i]);
    P(linear)(h1, io->cond_w2, NULL, B, D, 3 * D, cond_out);
    free(emb); free(h0); free(h1);
}

/* norm.rs:141-157 + :170 (LowRankAdaLn::forward, the modulation vectors):
 * (shift, scale, gate) = chunk(cond, 3); each += up(down(silu(.))) + b_up; gate -> tanh.
 * which: 0 = attention_adaln, 1 = mlp_adaln.  Outputs [B, D] each. */
void P(adaln_vectors)(const orc_cfg* c, const orc_block* blk, int which, const float* cond, int B,
                      float* shift, float* scale, float* gate) {
    int D = c->model_dim, r = c->adaln_rank;
    float* in = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* mid = (float*)malloc(sizeof(float) * (size_t)B * r);
    float* up = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* outs[3] = {shift, scale, gate};
    for (int ch = 0; ch < 3; ch++) {
        for (int b = 0; b < B; b++)
            for (int d = 0; d < D; d++)
                in[b * D + d] = (float)P(silu)((R)cond[(size_t)b * 3 * D + ch * D + d]);
        P(linear)(in, blk->ada_down[which][ch], NULL, B, D, r, mid);
        P(linear)(mid, blk->ada_up[which][ch], blk->ada_up_b[which][ch], B, r, D, up);
        for (int b = 0; b < B; b++)
            for (int d = 0; d < D; d++) {
                R v = (R)up[b * D + d] + (R)cond[(size_t)b * 3 * D + ch * D + d];
                outs[ch][b * D + d] = (float)(ch == 2 ? TANH(v) : v);
            }
    }
    free(in); free(mid); free(up);
}

/* A block GEMM y[M,N] = x[M,K] @ w[K,N] (no bias), in fp8 operands when c->gemm_fp8
 * (oracle.c): x quantized per row and 32-wide k block, w per output channel; the product
 * of the dequantized x and the unscaled weight codes, then times the channel scale. */
static void P(glinear)(const orc_cfg* c, const float* x, const float* w, int M, int K, int N, float* y) {
    if (!c || !c->gemm_fp8) {
        P(linear)(x, w, NULL, M, K, N, y);
        return;
    }
    uint8_t* qx = (uint8_t*)malloc((size_t)M * K);
    uint8_t* sx = (uint8_t*)malloc((size_t)M * (K / 32));
    uint8_t* qw = (uint8_t*)malloc((size_t)K * N);
    float* xd = (float*)malloc(sizeof(float) * (size_t)M * K);
    float* wd = (float*)malloc(sizeof(float) * (size_t)K * N);
    float* sw = (float*)malloc(sizeof(float) * (size_t)N);
    orc_mx_quantize_rows(x, M, K, qx, sx);
    orc_mx_dequantize_rows(qx, sx, M, K, xd);
    orc_quant_weight_cols(w, K, N, qw, sw);
    for (size_t i = 0; i < (size_t)K * N; i++) wd[i] = orc_e4m3_decode(qw[i]);
    P(linear)(xd, wd, NULL, M, K, N, y);
    for (int i = 0; i < M; i++)
        for (int n = 0; n < N; n++) y[(size_t)i * N + n] = (float)((R)y[(size_t)i * N + n] * (R)sw[n]);
    free(qx); free(sx); free(qw); free(xd); free(wd); free(sw);
}

/* The input of a GEMM that reads an adaLN output h = x r (1 + scale) + shift (norm.rs:160-169):
 * h itself, or (c->fused_adaln) its parts: xs = x (1 + scale) [M, K], r [M] and the shift rows
 * [B, K] of the B batch rows of S tokens each. */
typedef struct P(adaln_in) {
    const float* h;
    const float* xs;
    const float* r;
    const float* shift;
    int B, S;
} P(adaln_in);

/* y = h @ w, or for the folded form y = r (xs @ w) + shift_b @ w — each product a block GEMM
 * (glinear: in fp8 mode xs and the shift rows are quantized as GEMM inputs). */
static void P(glinear_in)(const orc_cfg* c, const P(adaln_in)* in, const float* w, int M, int K, int N,
                          float* y) {
    if (!in->xs) {
        P(glinear)(c, in->h, w, M, K, N, y);
        return;
    }
    float* ys = (float*)malloc(sizeof(float) * (size_t)in->B * N);
    P(glinear)(c, in->xs, w, M, K, N, y);
    P(glinear)(c, in->shift, w, in->B, K, N, ys);
    for (int i = 0; i < M; i++) {
        const float* sb = ys + (size_t)(i / in->S) * N;
        for (int n = 0; n < N; n++)
            y[(size_t)i * N + n] = (float)((R)y[(size_t)i * N + n] * (R)in->r[i] + (R)sb[n]);
    }
    free(ys);
}

/* The folded adaLN's parts of x [B, S, D] for one modulation (norm.rs:160-169):
 * xs = x (1 + scale[b]), r = 1 / sqrt(mean(x^2) + eps) per row. */
static void P(adaln_parts)(const float* x, const float* scale, int B, int S, int D, float eps, float* xs,
                           float* r) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < B * S; i++) {
        const int b = i / S;
        const float* xr = x + (size_t)i * D;
        R ss = 0;
        for (int d = 0; d < D; d++) ss += (R)xr[d] * (R)xr[d];
        r[i] = (float)(R_C(1.0) / SQRT(ss / (R)D + (R)eps));
        for (int d = 0; d < D; d++) xs[(size_t)i * D + d] = (float)((R)xr[d] * (R_C(1.0) + (R)scale[(size_t)b * D + d]));
    }
}

void P(gemm_fp8)(const float* x, const float* w, int M, int K, int N, float* y) {
    orc_cfg c;
    memset(&c, 0, sizeof c);
    c.gemm_fp8 = 1;
    P(glinear)(&c, x, w, M, K, N, y);
}

/* feed_forward.rs:76-85 (SwiGlu::forward_fused): u = h @ [W1|W3];
 * out = (silu(u[:, :F]) * u[:, F:]) @ W2. */
static void P(swiglu_c)(const orc_cfg* c, const P(adaln_in)* in, const float* w13, const float* w2, int M, int D,
                        int F, float* out) {
    float* u = (float*)malloc(sizeof(float) * (size_t)M * 2 * F);
    float* m = (float*)malloc(sizeof(float) * (size_t)M * F);
    P(glinear_in)(c, in, w13, M, D, 2 * F, u);
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++)
        for (int j = 0; j < F; j++)
            m[(size_t)i * F + j] =
                (float)(P(silu)((R)u[(size_t)i * 2 * F + j]) * (R)u[(size_t)i * 2 * F + F + j]);
    P(glinear)(c, m, w2, M, F, D, out);
    free(u); free(m);
}

void P(swiglu)(const float* h, const float* w13, const float* w2, int M, int D, int F,
               float* out) {
    P(adaln_in) in = {h, NULL, NULL, NULL, 0, 0};
    P(swiglu_c)(NULL, &in, w13, w2, M, D, F, out);
}

/* attention.rs:272-425 (JointAttention::forward_fused with a KV cache):
 *   [q|k|v] = h @ W_qkv; q = rope_half(q_norm(q)); k = rope_half(k_norm(k));
 *   K = [k | ctx_k], V = [v | ctx_v], mask = latent_mask ++ ctx_mask with latent_mask all
 *   ones when absent (build_joint_mask, attention.rs:730-750);
 *   o = SDPA(q, K, V, mask, Dh^-0.5); out = (sigmoid(h @ W_gate) * o) @ W_o.
 * ctx_k/ctx_v: [B, T, H, Dh] (already k-normed, not rotated); ctx_mask: [B, T] (1 = attend). */
static void P(joint_attention_in)(const orc_cfg* c, const orc_block* blk, const P(adaln_in)* in, int B,
                                  int S, int T, const float* ctx_k, const float* ctx_v,
                                  const uint8_t* ctx_mask, const uint8_t* lat_mask, const float* cos_t,
                                  const float* sin_t, float* out);
void P(joint_attention)(const orc_cfg* c, const orc_block* blk, const float* h, int B, int S,
                        int T, const float* ctx_k, const float* ctx_v, const uint8_t* ctx_mask,
                        const uint8_t* lat_mask, const float* cos_t, const float* sin_t, float* out) {
    P(adaln_in) in = {h, NULL, NULL, NULL, B, S};
    P(joint_attention_in)(c, blk, &in, B, S, T, ctx_k, ctx_v, ctx_mask, lat_mask, cos_t, sin_t, out);
}
static void P(joint_attention_in)(const orc_cfg* c, const orc_block* blk, const P(adaln_in)* in, int B,
                                  int S, int T, const float* ctx_k, const float* ctx_v,
                                  const uint8_t* ctx_mask, const uint8_t* lat_mask, const float* cos_t,
                                  const float* sin_t, float* out) {
    int D = c->model_dim, H = c->num_heads, Dh = c->head_dim, HD = H * Dh;
    int M = B * S, Skv = S + T;
    size_t szq = (size_t)M * HD;
    float* qkv = (float*)malloc(sizeof(float) * (size_t)M * 3 * HD);
    float* q = (float*)malloc(sizeof(float) * szq);
    float* kk = (float*)malloc(sizeof(float) * szq);
    float* vv = (float*)malloc(sizeof(float) * szq);
    float* tmp = (float*)malloc(sizeof(float) * szq);
    P(glinear_in)(c, in, blk->w_qkv, M, D, 3 * HD, qkv);
    for (int i = 0; i < M; i++)
        for (int j = 0; j < HD; j++) {
            q[(size_t)i * HD + j] = qkv[(size_t)i * 3 * HD + j];
            kk[(size_t)i * HD + j] = qkv[(size_t)i * 3 * HD + HD + j];
            vv[(size_t)i * HD + j] = qkv[(size_t)i * 3 * HD + 2 * HD + j];
        }
    P(head_rms_norm)(q, blk->q_norm, M, H, Dh, c->norm_eps, tmp);
    P(rope_half)(tmp, cos_t, sin_t, B, S, H, Dh, q);
    P(head_rms_norm)(kk, blk->k_norm, M, H, Dh, c->norm_eps, tmp);
    P(rope_half)(tmp, cos_t, sin_t, B, S, H, Dh, kk);

    /* Rearrange to [B, H, S(kv), Dh] (attention.rs:629-633 swap_dims). */
    float* qh = (float*)malloc(sizeof(float) * szq);
    float* kh = (float*)malloc(sizeof(float) * (size_t)B * H * Skv * Dh);
    float* vh = (float*)malloc(sizeof(float) * (size_t)B * H * Skv * Dh);
    float* mk = (float*)malloc(sizeof(float) * (size_t)B * Skv);
    float* oh = (float*)malloc(sizeof(float) * szq);
    for (int b = 0; b < B; b++)
        for (int hh = 0; hh < H; hh++) {
            for (int s = 0; s < S; s++)
                for (int d = 0; d < Dh; d++) {
                    size_t src = (((size_t)b * S + s) * H + hh) * Dh + d;
                    qh[(((size_t)b * H + hh) * S + s) * Dh + d] = q[src];
                    kh[(((size_t)b * H + hh) * Skv + s) * Dh + d] = kk[src];
                    vh[(((size_t)b * H + hh) * Skv + s) * Dh + d] = vv[src];
                }
            for (int j = 0; j < T; j++)
                for (int d = 0; d < Dh; d++) {
                    size_t src = (((size_t)b * T + j) * H + hh) * Dh + d;
                    kh[(((size_t)b * H + hh) * Skv + S + j) * Dh + d] = ctx_k[src];
                    vh[(((size_t)b * H + hh) * Skv + S + j) * Dh + d] = ctx_v[src];
                }
        }
    for (int b = 0; b < B; b++) {
        for (int s = 0; s < S; s++)
            mk[(size_t)b * Skv + s] = (lat_mask && !lat_mask[(size_t)b * S + s]) ? 0.0f : 1.0f;
        for (int j = 0; j < T; j++) mk[(size_t)b * Skv + S + j] = ctx_mask[(size_t)b * T + j] ? 1.0f : 0.0f;
    }
    P(sdpa)(qh, kh, vh, mk, B, H, S, Skv, Dh, (float)(R_C(1.0) / SQRT((R)Dh)), oh);

    /* gated = sigmoid(h @ W_gate) * o  (o back to [B, S, H*Dh]); out = gated @ W_o. */
    P(glinear_in)(c, in, blk->w_gate, M, D, D, tmp);
    for (int b = 0; b < B; b++)
        for (int s = 0; s < S; s++)
            for (int hh = 0; hh < H; hh++)
                for (int d = 0; d < Dh; d++) {
                    size_t dst = (((size_t)b * S + s) * H + hh) * Dh + d;
                    R o = (R)oh[(((size_t)b * H + hh) * S + s) * Dh + d];
                    q[dst] = (float)(P(sigmoid)((R)tmp[dst]) * o);
                }
    P(glinear)(c, q, blk->w_o, M, HD, D, out);
    free(qkv); free(q); free(kk); free(vv); free(tmp);
    free(qh); free(kh); free(vh); free(mk); free(oh);
}

/* diffusion.rs:62-105 (DiffusionBlock::forward_fused), dropout = identity:
 *   (h1, g1) = attention_adaln(x, c); x += g1 * JointAttention(h1)
 *   (h2, g2) = mlp_adaln(x, c);       x += g2 * SwiGLU(h2)
 * x: [B, S, D] updated in place; cond: [B, 3D]. */
void P(block_forward)(const orc_cfg* c, const orc_block* blk, float* x, const float* cond, int B,
                      int S, int T, const float* ctx_k, const float* ctx_v,
                      const uint8_t* ctx_mask, const uint8_t* lat_mask, const float* cos_t,
                      const float* sin_t) {
    int D = c->model_dim, F = c->mlp_hidden, M = B * S;
    size_t n = (size_t)M * D;
    float* shift = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* scale = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* gate = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* h = (float*)malloc(sizeof(float) * n);
    float* y = (float*)malloc(sizeof(float) * n);

    /* c->fused_adaln: the adaLN folded into the GEMMs that read h (orc_cfg), h never formed. */
    float* r = c->fused_adaln ? (float*)malloc(sizeof(float) * (size_t)M) : NULL;
    P(adaln_in) in = {h, c->fused_adaln ? h : NULL, r, shift, B, S};
    P(adaln_vectors)(c, blk, 0, cond, B, shift, scale, gate);
    if (c->fused_adaln) P(adaln_parts)(x, scale, B, S, D, c->norm_eps, h, r);
    else P(fused_adaln)(x, scale, shift, B, S, D, c->norm_eps, h);
    P(joint_attention_in)(c, blk, &in, B, S, T, ctx_k, ctx_v, ctx_mask, lat_mask, cos_t, sin_t, y);
    for (size_t i = 0; i < n; i++) {
        int b = (int)(i / ((size_t)S * D)), d = (int)(i % D);
        x[i] = (float)((R)x[i] + (R)gate[b * D + d] * (R)y[i]);
    }
    P(adaln_vectors)(c, blk, 1, cond, B, shift, scale, gate);
    if (c->fused_adaln) P(adaln_parts)(x, scale, B, S, D, c->norm_eps, h, r);
    else P(fused_adaln)(x, scale, shift, B, S, D, c->norm_eps, h);
    P(swiglu_c)(c, &in, blk->w13, blk->w2, M, D, F, y);
    for (size_t i = 0; i < n; i++) {
        int b = (int)(i / ((size_t)S * D)), d = (int)(i % D);
        x[i] = (float)((R)x[i] + (R)gate[b * D + d] * (R)y[i]);
    }
    free(shift); free(scale); free(gate); free(h); free(y); free(r);
}

/* dit/model.rs:354-393 (forward_backbone_fused) with per-layer cached context KV
 * (dit/model.rs:229-262):  c = cond_module(t); x = in_proj(x_t); 12 blocks;
 * v = out_proj(out_norm(x)).
 * ctx_k/ctx_v: [L][B][T][H][Dh]; ctx_mask: [B][T].
 * debug (nullable): [L+1][B][S][D] = after_in_proj then each block output
 * (BlockDebugOutputs, dit/model.rs:92-102). */
void P(forward)(const orc_cfg* c, const orc_io* io, const orc_block* blocks, int B, int S,
                const float* x_t, const float* t, int T, const float* ctx_k, const float* ctx_v,
                const uint8_t* ctx_mask, const uint8_t* lat_mask, float* v_out, float* debug) {
    int D = c->model_dim, Pd = c->latent_dim, L = c->num_layers, H = c->num_heads,
        Dh = c->head_dim;
    size_t n = (size_t)B * S * D, lay = (size_t)B * T * H * Dh;
    float* cond = (float*)malloc(sizeof(float) * (size_t)B * 3 * D);
    float* x = (float*)malloc(sizeof(float) * n);
    float* xn = (float*)malloc(sizeof(float) * n);
    float* cs = (float*)malloc(sizeof(float) * (size_t)S * (Dh / 2));
    float* sn = (float*)malloc(sizeof(float) * (size_t)S * (Dh / 2));
    P(rope_tables)(S, Dh, c->rope_theta, cs, sn);
    P(cond_module)(c, io, t, B, cond);
    P(linear)(x_t, io->in_w, io->in_b, B * S, Pd, D, x);
    if (debug) memcpy(debug, x, sizeof(float) * n);
    for (int l = 0; l < L; l++) {
        P(block_forward)(c, &blocks[l], x, cond, B, S, T, ctx_k + l * lay, ctx_v + l * lay,
                         ctx_mask, lat_mask, cs, sn);
        if (debug) memcpy(debug + (size_t)(l + 1) * n, x, sizeof(float) * n);
    }
    P(rms_norm)(x, io->out_norm_w, B * S, D, c->norm_eps, xn);
    P(linear)(xn, io->out_w, io->out_b, B * S, D, Pd, v_out);
    free(cond); free(x); free(xn); free(cs); free(sn);
}

/* attention.rs:431-501 (JointAttention::build_kv_cache): k_text = k_norm(text @ Wk_text),
 * v_text = text @ Wv_text, same for the aux (speaker) state; ctx = [text | aux] along seq,
 * ctx_mask = [text_mask | aux_mask].  aux may be NULL (Ta = 0).  Outputs [B, Tt+Ta, H, Dh]. */
void P(build_kv_cache)(const orc_cfg* c, const float* k_norm, int B, const float* text,
                       const uint8_t* text_mask, int Tt, int Dt, const float* wk_text,
                       const float* wv_text, const float* aux, const uint8_t* aux_mask, int Ta,
                       int Da, const float* wk_aux, const float* wv_aux, float* ctx_k,
                       float* ctx_v, uint8_t* ctx_mask) {
    int H = c->num_heads, Dh = c->head_dim, HD = H * Dh, T = Tt + (aux ? Ta : 0);
    for (int seg = 0; seg < 2; seg++) {
        const float* st = seg == 0 ? text : aux;
        int Ts = seg == 0 ? Tt : Ta, Ds = seg == 0 ? Dt : Da, off = seg == 0 ? 0 : Tt;
        const float* wk = seg == 0 ? wk_text : wk_aux;
        const float* wv = seg == 0 ? wv_text : wv_aux;
        const uint8_t* ms = seg == 0 ? text_mask : aux_mask;
        if (!st || Ts == 0) continue;
        float* kr = (float*)malloc(sizeof(float) * (size_t)B * Ts * HD);
        float* kn = (float*)malloc(sizeof(float) * (size_t)B * Ts * HD);
        float* vr = (float*)malloc(sizeof(float) * (size_t)B * Ts * HD);
        P(linear)(st, wk, NULL, B * Ts, Ds, HD, kr);
        P(head_rms_norm)(kr, k_norm, B * Ts, H, Dh, c->norm_eps, kn);
        P(linear)(st, wv, NULL, B * Ts, Ds, HD, vr);
        for (int b = 0; b < B; b++)
            for (int j = 0; j < Ts; j++) {
                memcpy(ctx_k + ((size_t)b * T + off + j) * HD, kn + ((size_t)b * Ts + j) * HD,
                       sizeof(float) * HD);
                memcpy(ctx_v + ((size_t)b * T + off + j) * HD, vr + ((size_t)b * Ts + j) * HD,
                       sizeof(float) * HD);
                ctx_mask[(size_t)b * T + off + j] = ms ? ms[(size_t)b * Ts + j] : 1;
            }
        free(kr); free(kn); free(vr);
    }
}

/* euler_sampler.rs:132-718, Joint-CFG Euler branch (:325-328, :379, :435-469, :565-566, :714):
 *   t_i = 0.999 (1 - i/N);  CFG iff min_t <= t_i <= max_t;
 *   v_c = forward(x, t_i, cond KV); v_u = forward(x, t_i, uncond KV);
 *   v = v_c + scale (v_c - v_u);  x += v (t_{i+1} - t_i).
 * Two separate B=U forwards, exactly as the reference runs them.  lat_mask (nullable,
 * [U, S]) masks latent keys of both forwards of utterance u (padded batches).  Runs at most
 * max_steps_run steps (<= 0: all); returns the number of steps run. */
int P(sample_joint_cfg)(const orc_cfg* c, const orc_io* io, const orc_block* blocks, int U,
                        int S, const float* x0, int T, const float* ctx_k_cond,
                        const float* ctx_v_cond, const uint8_t* mask_cond,
                        const float* ctx_k_unc, const float* ctx_v_unc, const uint8_t* mask_unc,
                        const uint8_t* lat_mask, int num_steps, float scale, float min_t,
                        float max_t, int max_steps_run, float* x_out) {
    int Pd = c->latent_dim;
    size_t n = (size_t)U * S * Pd;
    float* vc = (float*)malloc(sizeof(float) * n);
    float* vu = (float*)malloc(sizeof(float) * n);
    float* tt = (float*)malloc(sizeof(float) * (size_t)U);
    memcpy(x_out, x0, sizeof(float) * n);
    int run = (max_steps_run > 0 && max_steps_run < num_steps) ? max_steps_run : num_steps;
    for (int i = 0; i < run; i++) {
        /* The schedule is computed in f32 in the reference (euler_sampler.rs:326-328). */
        float t = 0.999f * (1.0f - (float)i / (float)num_steps);
        float tn = 0.999f * (1.0f - (float)(i + 1) / (float)num_steps);
        for (int u = 0; u < U; u++) tt[u] = t;
        int use_cfg = (min_t <= t) && (t <= max_t);
        P(forward)(c, io, blocks, U, S, x_out, tt, T, ctx_k_cond, ctx_v_cond, mask_cond, lat_mask, vc, NULL);
        if (use_cfg)
            P(forward)(c, io, blocks, U, S, x_out, tt, T, ctx_k_unc, ctx_v_unc, mask_unc, lat_mask, vu, NULL);
        float dt = tn - t;
        for (size_t j = 0; j < n; j++) {
            R v = (R)vc[j];
            if (use_cfg) v = v + ((R)vc[j] - (R)vu[j]) * (R)scale;
            x_out[j] = (float)((R)x_out[j] + v * (R)dt);
        }
    }
    free(vc); free(vu); free(tt);
    return run;
}

/* Active CFG signals in the reference's order (euler_sampler.rs:163-200): text if its
 * scale is > 0; speaker if the model uses speaker conditioning, the condition holds a
 * speaker state and its scale is > 0; caption if the condition holds a caption with a
 * valid token and its scale is > 0.  scales[k] = scale of signal k; returns the count. */
static int P(cfg_signals)(const orc_sampler* sp, float* scales) {
    int n = 0;
    if (sp->scale_text > 0.f) scales[n++] = sp->scale_text;
    if (sp->has_speaker && sp->scale_speaker > 0.f) scales[n++] = sp->scale_speaker;
    if (sp->has_caption && sp->scale_caption > 0.f) scales[n++] = sp->scale_caption;
    return n;
}

/* kv_scaling.rs:10-60 on the role copies: the aux keys [aux_start, T) of K and V of every
 * scaled role times s, in the first nl layers. */
static void P(scale_aux_kv)(float* const* rk, float* const* rv, const int* roles, int nroles,
                            int nl, int U, int T, int HD, int aux_start, float s) {
    for (int ri = 0; ri < nroles; ri++)
        for (int l = 0; l < nl; l++)
            for (int u = 0; u < U; u++)
                for (int j = aux_start; j < T; j++) {
                    size_t o = (((size_t)l * U + u) * T + j) * HD;
                    for (int e = 0; e < HD; e++) {
                        rk[roles[ri]][o + e] = (float)((R)rk[roles[ri]][o + e] * (R)s);
                        rv[roles[ri]][o + e] = (float)((R)rv[roles[ri]][o + e] * (R)s);
                    }
                }
}

/* math.rs:38-53 temporal_score_rescale (no-op for t >= 1): with 1-t = omt,
 * snr = omt^2 / t^2, ratio = (snr sigma^2 + 1) / (snr sigma^2 / k + 1),
 * v' = (v omt + x) ratio / omt - x / omt.  The scalars are f32, as in the reference. */
static void P(temporal_rescale)(float* v, const float* x, size_t n, float t, float k, float sigma) {
    if (t >= 1.0f) return;
    float omt = 1.0f - t;
    float snr = (omt * omt) / (t * t);
    float sig2 = sigma * sigma;
    float ratio = (snr * sig2 + 1.0f) / (snr * sig2 / k + 1.0f);
    for (size_t j = 0; j < n; j++) {
        R a = (R)v[j] * (R)omt + (R)x[j];
        v[j] = (float)(a * (R)ratio / (R)omt - (R)x[j] / (R)omt);
    }
}

/* The guided velocity at (x, t) (euler_sampler.rs:435-523 and the Heun corrector's copy
 * :571-666): the conditioned forward (role 0), and when CFG is on
 *   Independent  v = v_c; v += (v_c - v_k) s_k for every enabled signal k (role 1 + k),
 *   Joint        v = v_c + (v_c - v_u) s_0 (role 1),
 *   Alternating  a = i mod n: v = v_c + (v_c - v_a) s_a (role 1 + a).
 * rk/rv/rm hold one [L, U, T, H, Dh] / [U, T] copy per role. */
static void P(guided_velocity)(const orc_cfg* c, const orc_io* io, const orc_block* blocks,
                               int U, int S, const float* x, float t, int use_cfg, int step,
                               int mode, int n, const float* scales, int T,
                               float* const* rk, float* const* rv, uint8_t* const* rm,
                               const uint8_t* lat_mask, float* tt, float* vtmp, float* v) {
    size_t nel = (size_t)U * S * c->latent_dim;
    for (int u = 0; u < U; u++) tt[u] = t;
    P(forward)(c, io, blocks, U, S, x, tt, T, rk[0], rv[0], rm[0], lat_mask, v, NULL);
    if (!use_cfg) return;
    if (mode == 0) {
        float* vc = vtmp + nel * n;  /* keep v_c while v accumulates */
        memcpy(vc, v, sizeof(float) * nel);
        for (int k = 0; k < n; k++)
            P(forward)(c, io, blocks, U, S, x, tt, T, rk[1 + k], rv[1 + k], rm[1 + k], lat_mask,
                       vtmp + nel * k, NULL);
        for (size_t j = 0; j < nel; j++) {
            R acc = (R)vc[j];
            for (int k = 0; k < n; k++) acc = acc + ((R)vc[j] - (R)vtmp[nel * k + j]) * (R)scales[k];
            v[j] = (float)acc;
        }
    } else {
        int a = mode == 1 ? 0 : step % n;
        P(forward)(c, io, blocks, U, S, x, tt, T, rk[1 + a], rv[1 + a], rm[1 + a], lat_mask, vtmp, NULL);
        for (size_t j = 0; j < nel; j++) v[j] = (float)((R)v[j] + ((R)v[j] - (R)vtmp[j]) * (R)scales[a]);
    }
}

/* euler_sampler.rs:132-718 — the RF ODE loop with CFG, every mode and integrator:
 *   x = noise (times truncation_factor); t_i = 0.999 (1 - i/N) in f32 (:325-328);
 *   CFG at t iff a signal is enabled and min_t <= t <= max_t (:379);
 *   v1 = guided velocity at (x, t_i) (guided_velocity), temporally rescaled (:525-530);
 *   the speaker-KV scaling reverts once t_{i+1} < min_t <= t_i, before the corrector (:533-545);
 *   Euler  x += v1 dt;
 *   Heun   x_p = x + v1 dt, v2 = guided velocity at (x_p, t_{i+1}) with the same dropped
 *          condition index i, rescaled at t_{i+1}; x += (v1 + v2) / 2 dt (:567-683);
 *   PLMS-4 the newest-first history of v1 (at most 4) is cleared whenever (CFG on,
 *          speaker KV active) changes between steps (:341-347, :383-390); Adams-Bashforth
 *          orders 1-4 (:98-117); x += v_eff dt (:714).
 * ctx_k/ctx_v [L, R*U, T, H, Dh], ctx_mask [R*U, T] are role-major: role r of utterance u
 * is row r*U + u, with role 0 the conditioned bundle, Joint role 1 the unconditioned one,
 * and Independent / Alternating role 1+k the bundle with enabled signal k dropped
 * (make_single_uncond, :41-85).  Speaker-KV scaling (kv_scaling.rs:10-60) multiplies the
 * aux keys of role 0, and of every role in Independent mode (the batched cache), in the
 * first max_layers layers.  lat_mask (nullable, [U, S]) masks latent keys in every forward.
 * Runs at most max_steps_run steps (<= 0: all); returns the number run. */
int P(sample_rf)(const orc_cfg* c, const orc_io* io, const orc_block* blocks, int U, int S,
                 const float* x0, int T, const float* ctx_k, const float* ctx_v,
                 const uint8_t* ctx_mask, const uint8_t* lat_mask, const orc_sampler* sp,
                 int max_steps_run, float* x_out) {
    const int L = c->num_layers, HD = c->num_heads * c->head_dim, Pd = c->latent_dim;
    const int N = sp->num_steps;
    float scales[3];
    const int n = P(cfg_signals)(sp, scales);
    const int Rr = sp->cfg_mode == 1 ? (n > 0 ? 2 : 1) : 1 + n;  /* roles */
    const size_t nel = (size_t)U * S * Pd, lay = (size_t)T * HD;
    float* rk[4];
    float* rv[4];
    uint8_t* rm[4];
    for (int r = 0; r < Rr; r++) {
        rk[r] = (float*)malloc(sizeof(float) * L * U * lay);
        rv[r] = (float*)malloc(sizeof(float) * L * U * lay);
        rm[r] = (uint8_t*)malloc((size_t)U * T);
        for (int l = 0; l < L; l++)
            for (int u = 0; u < U; u++) {
                size_t src = ((size_t)l * Rr * U + (size_t)r * U + u) * lay;
                memcpy(rk[r] + ((size_t)l * U + u) * lay, ctx_k + src, sizeof(float) * lay);
                memcpy(rv[r] + ((size_t)l * U + u) * lay, ctx_v + src, sizeof(float) * lay);
            }
        memcpy(rm[r], ctx_mask + (size_t)r * U * T, (size_t)U * T);
    }
    int scaled_roles[4], nsr = 0;
    scaled_roles[nsr++] = 0;
    if (sp->cfg_mode == 0)
        for (int r = 1; r < Rr; r++) scaled_roles[nsr++] = r;
    const int nl = sp->speaker_kv_max_layers < 0 || sp->speaker_kv_max_layers > L ? L : sp->speaker_kv_max_layers;
    int spk_active = sp->has_speaker_kv != 0;
    if (spk_active && sp->has_speaker)
        P(scale_aux_kv)(rk, rv, scaled_roles, nsr, nl, U, T, HD, sp->ctx_aux_start, sp->speaker_kv_scale);

    float* ts = (float*)malloc(sizeof(float) * (N + 1));
    for (int i = 0; i <= N; i++) ts[i] = 0.999f * (1.0f - (float)i / (float)N);
    float* v1 = (float*)malloc(sizeof(float) * nel);
    float* v2 = (float*)malloc(sizeof(float) * nel);
    float* xp = (float*)malloc(sizeof(float) * nel);
    float* vtmp = (float*)malloc(sizeof(float) * nel * (n + 1 > 1 ? n + 1 : 1));
    float* hist = (float*)malloc(sizeof(float) * nel * 4);  /* hist[k] = k-th newest */
    float* tt = (float*)malloc(sizeof(float) * U);
    int nhist = 0;
    for (size_t j = 0; j < nel; j++) x_out[j] = sp->has_truncation ? (float)((R)x0[j] * (R)sp->truncation_factor) : x0[j];
    int prev_cfg = n > 0 && sp->min_t <= ts[0] && ts[0] <= sp->max_t, prev_spk = spk_active;
    const int run = (max_steps_run > 0 && max_steps_run < N) ? max_steps_run : N;
    for (int i = 0; i < run; i++) {
        const float t = ts[i], tn = ts[i + 1];
        const int use_cfg = n > 0 && sp->min_t <= t && t <= sp->max_t;
        if (sp->method == 2 && (use_cfg != prev_cfg || spk_active != prev_spk)) {
            nhist = 0;
            prev_cfg = use_cfg;
            prev_spk = spk_active;
        }
        P(guided_velocity)(c, io, blocks, U, S, x_out, t, use_cfg, i, sp->cfg_mode, n, scales, T,
                           rk, rv, rm, lat_mask, tt, vtmp, v1);
        if (sp->has_temporal_rescale) P(temporal_rescale)(v1, x_out, nel, t, sp->rescale_k, sp->rescale_sigma);
        if (spk_active && sp->has_speaker && sp->speaker_kv_has_min_t && tn < sp->speaker_kv_min_t &&
            t >= sp->speaker_kv_min_t) {
            P(scale_aux_kv)(rk, rv, scaled_roles, nsr, nl, U, T, HD, sp->ctx_aux_start, 1.0f / sp->speaker_kv_scale);
            spk_active = 0;
        }
        const float dt = tn - t;
        if (sp->method == 1) {
            for (size_t j = 0; j < nel; j++) xp[j] = (float)((R)x_out[j] + (R)v1[j] * (R)dt);
            const int use_cfg2 = n > 0 && sp->min_t <= tn && tn <= sp->max_t;
            P(guided_velocity)(c, io, blocks, U, S, xp, tn, use_cfg2, i, sp->cfg_mode, n, scales, T,
                               rk, rv, rm, lat_mask, tt, vtmp, v2);
            if (sp->has_temporal_rescale) P(temporal_rescale)(v2, xp, nel, tn, sp->rescale_k, sp->rescale_sigma);
            for (size_t j = 0; j < nel; j++) {
                R ve = ((R)v1[j] + (R)v2[j]) / R_C(2.0);
                x_out[j] = (float)((R)x_out[j] + ve * (R)dt);
            }
        } else if (sp->method == 2) {
            for (int k = (nhist < 4 ? nhist : 3); k > 0; k--) memcpy(hist + nel * k, hist + nel * (k - 1), sizeof(float) * nel);
            memcpy(hist, v1, sizeof(float) * nel);
            nhist = nhist < 4 ? nhist + 1 : 4;
            for (size_t j = 0; j < nel; j++) {
                R ve;
                const R h0 = (R)hist[j];
                if (nhist == 1) {
                    ve = h0;
                } else if (nhist == 2) {
                    ve = h0 * (R)1.5f + (R)hist[nel + j] * (R)-0.5f;
                } else if (nhist == 3) {
                    ve = h0 * (R)(23.0f / 12.0f) + (R)hist[nel + j] * (R)(-16.0f / 12.0f) +
                         (R)hist[2 * nel + j] * (R)(5.0f / 12.0f);
                } else {
                    ve = h0 * (R)(55.0f / 24.0f) + (R)hist[nel + j] * (R)(-59.0f / 24.0f) +
                         (R)hist[2 * nel + j] * (R)(37.0f / 24.0f) + (R)hist[3 * nel + j] * (R)(-9.0f / 24.0f);
                }
                x_out[j] = (float)((R)x_out[j] + ve * (R)dt);
            }
        } else {
            for (size_t j = 0; j < nel; j++) x_out[j] = (float)((R)x_out[j] + (R)v1[j] * (R)dt);
        }
    }
    for (int r = 0; r < Rr; r++) { free(rk[r]); free(rv[r]); free(rm[r]); }
    free(ts); free(v1); free(v2); free(xp); free(vtmp); free(hist); free(tt);
    return run;
}

/* TextBlock::forward (text_encoder.rs:46-60), dropout = identity:
 *   a = SelfAttention(attention_norm(x)); x += a;  x += SwiGlu(mlp_norm(x)).
 * SelfAttention (attention.rs:96-121): q, k, v = h @ Wq, Wk, Wv -> [B, S, H, Dh];
 * q, k head-RMSNormed (q_norm / k_norm), full RoPE on every head (rope.rs:82-113);
 * o = SDPA(q, k, v, key mask, Dh^-0.5); out = (o * sigmoid(h @ W_gate)) @ Wo.
 * x [B, S, E] in place; mask [B, S] (nonzero = valid key). */
void P(text_block)(const orc_enc_cfg* c, const orc_enc_block* blk, float* x, const uint8_t* mask, int B,
                   int S, const float* cos_t, const float* sin_t) {
    const int E = c->dim, H = c->num_heads, Dh = E / H, HD = H * Dh, F = c->mlp_hidden, M = B * S;
    const size_t n = (size_t)M * E, nq = (size_t)M * HD;
    float* h = (float*)malloc(sizeof(float) * n);
    float* q = (float*)malloc(sizeof(float) * nq);
    float* k = (float*)malloc(sizeof(float) * nq);
    float* v = (float*)malloc(sizeof(float) * nq);
    float* t = (float*)malloc(sizeof(float) * nq);
    float* qh = (float*)malloc(sizeof(float) * nq);
    float* kh = (float*)malloc(sizeof(float) * nq);
    float* vh = (float*)malloc(sizeof(float) * nq);
    float* oh = (float*)malloc(sizeof(float) * nq);
    float* g = (float*)malloc(sizeof(float) * n);
    float* mk = (float*)malloc(sizeof(float) * (size_t)B * S);
    float* y = (float*)malloc(sizeof(float) * n);
    P(rms_norm)(x, blk->attn_norm, M, E, c->norm_eps, h);
    P(linear)(h, blk->wq, NULL, M, E, HD, q);
    P(linear)(h, blk->wk, NULL, M, E, HD, k);
    P(linear)(h, blk->wv, NULL, M, E, HD, v);
    P(head_rms_norm)(q, blk->q_norm, M, H, Dh, c->norm_eps, t);
    P(rope_full)(t, cos_t, sin_t, B, S, H, Dh, q);
    P(head_rms_norm)(k, blk->k_norm, M, H, Dh, c->norm_eps, t);
    P(rope_full)(t, cos_t, sin_t, B, S, H, Dh, k);
    for (int b = 0; b < B; b++)
        for (int hh = 0; hh < H; hh++)
            for (int s = 0; s < S; s++)
                for (int d = 0; d < Dh; d++) {
                    const size_t src = (((size_t)b * S + s) * H + hh) * Dh + d;
                    const size_t dst = (((size_t)b * H + hh) * S + s) * Dh + d;
                    qh[dst] = q[src];
                    kh[dst] = k[src];
                    vh[dst] = v[src];
                }
    for (int i = 0; i < B * S; i++) mk[i] = mask[i] ? 1.f : 0.f;
    P(sdpa)(qh, kh, vh, mk, B, H, S, S, Dh, (float)(R_C(1.0) / SQRT((R)Dh)), oh);
    P(linear)(h, blk->w_gate, NULL, M, E, E, g);
    for (int b = 0; b < B; b++)
        for (int s = 0; s < S; s++)
            for (int hh = 0; hh < H; hh++)
                for (int d = 0; d < Dh; d++) {
                    const size_t dst = (((size_t)b * S + s) * H + hh) * Dh + d;
                    t[dst] = (float)((R)oh[(((size_t)b * H + hh) * S + s) * Dh + d] * P(sigmoid)((R)g[dst]));
                }
    P(linear)(t, blk->wo, NULL, M, HD, E, y);
    for (size_t i = 0; i < n; i++) x[i] = (float)((R)x[i] + (R)y[i]);
    P(rms_norm)(x, blk->mlp_norm, M, E, c->norm_eps, h);
    P(swiglu)(h, blk->w13, blk->w2, M, E, F, y);
    for (size_t i = 0; i < n; i++) x[i] = (float)((R)x[i] + (R)y[i]);
    free(h); free(q); free(k); free(v); free(t); free(qh); free(kh); free(vh); free(oh); free(g);
    free(mk); free(y);
}

/* A condition encoder and its conditioner norm:
 *   text / caption (TextEncoder::forward, text_encoder.rs:117-147): x = embedding[ids];
 *   speaker (ReferenceLatentEncoder::forward, speaker_encoder.rs:135-162):
 *     x = (latent @ in_w + in_b) / 6;
 *   then x *= mask; per block x = TextBlock(x), x *= mask; x *= mask;
 *   state = RmsNorm(out_norm)(x) (text_norm, dit/model.rs:189-190, or the speaker /
 *   caption conditioner's norm, aux_conditioner.rs:60-85);
 *   mean_token (speaker, prepend_masked_mean_token, aux_conditioner.rs:150-185): out =
 *   [sum_s mask * state / max(count, 1) | state], mask_out = [count > 0 | mask].
 * ids [B, S] (embedding != NULL) or latent [B, S, in_dim]; out [B, S + mean_token, E]. */
void P(encoder_forward)(const orc_enc_cfg* c, const orc_enc_block* blocks, const float* embedding,
                        const float* in_w, const float* in_b, int in_dim, const float* out_norm, int mean_token,
                        int B, int S, const int32_t* ids, const float* latent, const uint8_t* mask, float* out,
                        uint8_t* mask_out) {
    const int E = c->dim, Dh = E / c->num_heads, M = B * S;
    const size_t n = (size_t)M * E;
    float* x = (float*)malloc(sizeof(float) * n);
    float* st = (float*)malloc(sizeof(float) * n);
    float* cs = (float*)malloc(sizeof(float) * (size_t)S * (Dh / 2));
    float* sn = (float*)malloc(sizeof(float) * (size_t)S * (Dh / 2));
    if (embedding) {
        for (int i = 0; i < M; i++) memcpy(x + (size_t)i * E, embedding + (size_t)ids[i] * E, sizeof(float) * E);
    } else {
        P(linear)(latent, in_w, in_b, M, in_dim, E, x);
        for (size_t i = 0; i < n; i++) x[i] = (float)((R)x[i] / R_C(6.0));
    }
    for (int i = 0; i < M; i++)
        if (!mask[i]) memset(x + (size_t)i * E, 0, sizeof(float) * E);
    P(rope_tables)(S, Dh, 10000.f, cs, sn);
    for (int l = 0; l < c->num_layers; l++) {
        P(text_block)(c, &blocks[l], x, mask, B, S, cs, sn);
        for (int i = 0; i < M; i++)
            if (!mask[i]) memset(x + (size_t)i * E, 0, sizeof(float) * E);
    }
    P(rms_norm)(x, out_norm, M, E, c->norm_eps, st);
    const int T = S + (mean_token ? 1 : 0);
    for (int b = 0; b < B; b++) {
        float* ob = out + (size_t)b * T * E;
        if (mean_token) {
            int cnt = 0;
            for (int s = 0; s < S; s++) cnt += mask[(size_t)b * S + s] ? 1 : 0;
            const R den = cnt > 0 ? (R)cnt : R_C(1.0);
            for (int d = 0; d < E; d++) {
                R acc = 0;
                for (int s = 0; s < S; s++)
                    if (mask[(size_t)b * S + s]) acc += (R)st[((size_t)b * S + s) * E + d];
                ob[d] = (float)(acc / den);
            }
            if (mask_out) mask_out[(size_t)b * T] = cnt > 0;
        }
        memcpy(ob + (size_t)(T - S) * E, st + (size_t)b * S * E, sizeof(float) * (size_t)S * E);
        if (mask_out)
            for (int s = 0; s < S; s++) mask_out[(size_t)b * T + (T - S) + s] = mask[(size_t)b * S + s] ? 1 : 0;
    }
    free(x); free(st); free(cs); free(sn);
}

/* Conv1d (stride 1) on channels-first x [C, L]: y[o, t] = b[o] + sum_{c, j} w[o, c, j]
 * x[c, t + j dil - pad], zero outside [0, L); y [O, L_out], L_out = L + 2 pad - dil (k - 1)
 * (burn Conv1d with PaddingConfig1d::Explicit(pad, pad), layers.rs:70-93). */
void P(conv1d)(const float* x, int C, int L, const float* w, const float* b, int O, int k, int dil, int pad,
               float* y) {
    const int Lo = L + 2 * pad - dil * (k - 1);
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int t = 0; t < Lo; t++) {
            R acc = b ? (R)b[o] : R_C(0.0);
            for (int c = 0; c < C; c++)
                for (int j = 0; j < k; j++) {
                    const int src = t + j * dil - pad;
                    if (src >= 0 && src < L) acc += (R)w[((size_t)o * C + c) * k + j] * (R)x[(size_t)c * L + src];
                }
            y[(size_t)o * Lo + t] = (float)acc;
        }
}

/* ConvTranspose1d on x [C, L]: y[o, t] = b[o] + sum over (i, j) with i stride - pad + j = t
 * of w[c, o, j] x[c, i]; y [O, L_out], L_out = (L - 1) stride - 2 pad + k + pad_out
 * (weights.rs:80-103 with conv_transpose_pad, layers.rs:62-65). */
void P(conv_transpose1d)(const float* x, int C, int L, const float* w, const float* b, int O, int k, int stride,
                         int pad, int pad_out, float* y) {
    const int Lo = (L - 1) * stride - 2 * pad + k + pad_out;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int t = 0; t < Lo; t++) {
            R acc = b ? (R)b[o] : R_C(0.0);
            for (int j = 0; j < k; j++) {
                const int num = t + pad - j;
                if (num < 0 || num % stride) continue;
                const int i = num / stride;
                if (i >= L) continue;
                for (int c = 0; c < C; c++) acc += (R)w[((size_t)c * O + o) * k + j] * (R)x[(size_t)c * L + i];
            }
            y[(size_t)o * Lo + t] = (float)acc;
        }
}

/* Snake1d (layers.rs:24-31): y = x + sin(alpha x)^2 / (alpha + 1e-9), alpha per channel. */
void P(snake)(const float* x, const float* alpha, int C, int L, float* y) {
    for (int c = 0; c < C; c++) {
        const R a = (R)alpha[c];
        for (int t = 0; t < L; t++) {
            const R v = (R)x[(size_t)c * L + t];
            const R sv = SIN(a * v);
            y[(size_t)c * L + t] = (float)(v + sv * sv / (a + (R)1e-9f));
        }
    }
}

/* DacVaeCodec::decode (model.rs:33-38): latent [B, T, latent_dim] -> wav [B, T * hop],
 * hop = prod(rates); per row channels-first, as the reference. */
void P(codec_decode)(const orc_codec* cd, int B, int T, const float* latent, float* wav) {
    int hop = 1;
    for (int i = 0; i < cd->num_blocks; i++) hop *= cd->rates[i];
    size_t cap = (size_t)cd->decoder_dim * T;
    {
        int L = T, C = cd->decoder_dim;
        for (int i = 0; i < cd->num_blocks; i++) {
            L *= cd->rates[i];
            C /= 2;
            if ((size_t)C * L > cap) cap = (size_t)C * L;
        }
        if ((size_t)cd->proj_dim * T > cap) cap = (size_t)cd->proj_dim * T;
        if ((size_t)cd->latent_dim * T > cap) cap = (size_t)cd->latent_dim * T;  /* the transposed latent */
    }
    float* a = (float*)malloc(sizeof(float) * cap);
    float* b2 = (float*)malloc(sizeof(float) * cap);
    float* c2 = (float*)malloc(sizeof(float) * cap);
    for (int bb = 0; bb < B; bb++) {
        int L = T, C = cd->latent_dim;
        for (int ch = 0; ch < C; ch++)
            for (int t = 0; t < L; t++) a[(size_t)ch * L + t] = latent[((size_t)bb * T + t) * C + ch];
        P(conv1d)(a, C, L, cd->out_proj_w, cd->out_proj_b, cd->proj_dim, 1, 1, 0, b2);
        C = cd->proj_dim;
        P(conv1d)(b2, C, L, cd->stem_w, cd->stem_b, cd->decoder_dim, 7, 1, 3, a);
        C = cd->decoder_dim;
        for (int i = 0; i < cd->num_blocks; i++) {
            const orc_codec_block* bl = &cd->blocks[i];
            const int r = cd->rates[i], O = C / 2;
            P(snake)(a, bl->alpha, C, L, b2);
            P(conv_transpose1d)(b2, C, L, bl->convt_w, bl->convt_b, O, 2 * r, r, (r + 1) / 2, r % 2, a);
            L *= r;
            C = O;
            static const int dils[3] = {1, 3, 9};
            for (int u = 0; u < 3; u++) {
                P(snake)(a, bl->res_alpha0[u], C, L, b2);
                P(conv1d)(b2, C, L, bl->res_conv_w[u], bl->res_conv_b[u], C, 7, dils[u], 3 * dils[u], c2);
                P(snake)(c2, bl->res_alpha1[u], C, L, b2);
                P(conv1d)(b2, C, L, bl->res_pw_w[u], bl->res_pw_b[u], C, 1, 1, 0, c2);
                for (size_t e = 0; e < (size_t)C * L; e++) a[e] = (float)((R)a[e] + (R)c2[e]);
            }
        }
        P(snake)(a, cd->head_alpha, C, L, b2);
        P(conv1d)(b2, C, L, cd->head_w, cd->head_b, 1, 7, 1, 3, c2);
        for (int t = 0; t < L; t++) wav[(size_t)bb * L + t] = (float)TANH((R)c2[t]);
        (void)hop;
    }
    free(a); free(b2); free(c2);
}
