// libirodori_hip host side: the C ABI of include/irodori_hip.h.
//
// A context owns every device buffer of one model instance, sized once at creation:
//   weights   bf16 (or f32) K-major [N, K] for the four projection GEMMs, f32 for the
//             norms / conditioning MLPs;
//   context   per layer K/V [rows, H, max_ctx, Dh] + mask + per-64-key-tile "any valid"
//             flags (the CondKvCache of attention.rs:24-45, laid out for the attention
//             kernel's second key segment);
//   work      residual x f32 [rows*S, D], modulated h, Q/K/V of the latent keys,
//             sigmoid gate, gated attention output, SwiGLU product;
//   tables    RoPE cos/sin [max_seq, Dh/2], adaLN modulation vectors per (step, layer).
// One RF step is recorded once into a hipGraph and replayed num_steps times; the step
// index lives in device memory and is advanced by the last node of the graph.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <tuple>
#include <type_traits>
#include <vector>

#include "../../include/irodori_hip.h"
#include "common.hpp"
#include "kernels.hpp"
#include "roctx.hpp"
#include "host.hpp"

namespace irodori {

static thread_local std::string g_last_error;
void set_last_error(const std::string& msg) { g_last_error = msg; }

int tracked_alloc(std::vector<void*>& allocs, uint64_t& total, void** p, size_t bytes) {
    if (bytes == 0) bytes = 16;
    if (const char* lim = std::getenv("IRODORI_DEVICE_ALLOC_LIMIT")) {
        const unsigned long long limit = std::strtoull(lim, nullptr, 10);
        if (limit > 0 && total + bytes > limit) {
            set_last_error("device allocation of " + std::to_string(bytes) + " bytes would exceed "
                           "IRODORI_DEVICE_ALLOC_LIMIT (" + std::to_string(limit) + " bytes; " +
                           std::to_string(total) + " already held)");
            return IRODORI_ERR_OOM;
        }
    }
    allocs.push_back(nullptr);  // the slot first: a throwing push_back must not strand the allocation
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        allocs.pop_back();
        set_last_error(std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? IRODORI_ERR_OOM : IRODORI_ERR_HIP;
    }
    allocs.back() = *p;
    total += bytes;
    return IRODORI_OK;
}

}  // namespace irodori

using namespace irodori;

struct LayerBufs {
    void* w_qkvg = nullptr;  // [4D, D]
    void* w_o = nullptr;     // [D, HD]
    void* w13 = nullptr;     // [2F, D], W1/W3 rows interleaved per 32
    void* w2 = nullptr;      // [D, F]
    // fp8 compute: the four weights above hold e4m3 codes; their per-row (output channel)
    // scales.
    float* ws_qkvg = nullptr;
    float* ws_o = nullptr;
    float* ws_13 = nullptr;
    float* ws_2 = nullptr;
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    float* ada_down[2][3] = {};
    float* ada_up[2][3] = {};
    float* ada_up_b[2][3] = {};
    void* ctx_k = nullptr;   // [rows, H, max_ctx, Dh]
    void* ctx_v = nullptr;      // V^T [rows, H, Dh, Tp] (Tp = max_ctx rounded up to 64), keys permuted
    float* ctx_mask = nullptr;  // [rows, max_ctx]
    int* tile_on = nullptr;     // [rows, ceil(max_ctx / 64)]
    unsigned long long* tile_bits = nullptr;  // [rows, ceil(max_ctx / 64)], bit k: key 64 t + k valid
    // Context projections (wk/wv_text, wk/wv_speaker|caption, attention.rs:142-147): per
    // segment (0 text, 1 aux) [2 H Dh, kpad] = [Wk ; Wv]^T, input dim zero-padded to 64.
    void* w_ctx[2] = {};
    bool ctx_proj_loaded = false;
    bool loaded = false;
    std::vector<char> row_set;
};

// A captured RF step is specific to the batch shape, the context length and the CFG
// scale (a kernel argument baked into the graph).
// One captured sampler evaluation: the role chains it runs, the integrator phase, and
// what the captured kernels read (context length, latent masks, scaled speaker KV).
struct GraphKey {
    int U, S, T;
    int roles;          // bit r set: role r runs (rows r*U .. r*U + U - 1)
    int method, phase;
    int latent_masked;  // the captured attention reads the latent key masks
    int kv_scaled;      // layers whose captured attention reads the speaker-scaled copies
    bool operator<(const GraphKey& o) const {
        return std::tie(U, S, T, roles, method, phase, latent_masked, kv_scaled) <
               std::tie(o.U, o.S, o.T, o.roles, o.method, o.phase, o.latent_masked, o.kv_scaled);
    }
};

// Captured sampler graphs, least recently used first out beyond kMax (each executable holds
// its ~120 kernel nodes and their arguments; a server cycling through many utterance lengths
// would otherwise keep one per length).  An entry is only dropped on a cache miss, after the
// capture's stream synchronisation, so no dropped graph is still running.
struct GraphCache {
    static constexpr size_t kMax = 64;
    struct Entry {
        hipGraphExec_t exec;
        uint64_t last;
    };
    std::map<GraphKey, Entry> map;
    uint64_t tick = 0;
    hipGraphExec_t find(const GraphKey& k) {
        auto it = map.find(k);
        if (it == map.end()) return nullptr;
        it->second.last = ++tick;
        return it->second.exec;
    }
    void insert(const GraphKey& k, hipGraphExec_t e) {
        while (map.size() >= kMax) {
            auto old = map.begin();
            for (auto it = map.begin(); it != map.end(); ++it)
                if (it->second.last < old->second.last) old = it;
            (void)hipGraphExecDestroy(old->second.exec);
            map.erase(old);
        }
        map[k] = Entry{e, ++tick};
    }
    void clear() {
        for (auto& kv : map) (void)hipGraphExecDestroy(kv.second.exec);
        map.clear();
    }
    size_t size() const { return map.size(); }
};

struct irodori_ctx {
    int device = 0;
    irodori_dit_config cfg{};
    // SwiGLU hidden width on the device: mlp_hidden rounded up to 128 (whole GEMM tiles and
    // K slices).  The padding columns of W1 / W3 and rows of W2 are zero, so the padded
    // products are silu(0) * 0 = 0 and add nothing.
    int Fp = 0;
    bool bf16 = true;
    bool fp8 = false;  // block GEMMs on e4m3 operands (activations and attention stay bf16)
    // Block GEMM weights stored tile-major (GemmArgs::w_tiled): every row count is a multiple
    // of 64 and every row a multiple of 128 bytes (fp8 codes: D and H Dh multiples of 128).
    bool w_tiled = false;
    size_t esz = 2;    // compute element size
    hipStream_t stream = nullptr;
    // Side capture streams and fork/join events: a captured sampler evaluation runs each
    // CFG role as an independent chain of kernels (role 0 on `stream`) until the update.
    static constexpr int kMaxRoles = 3;
    hipStream_t side[kMaxRoles - 1] = {};
    hipEvent_t ev_fork = nullptr, ev_join[kMaxRoles - 1] = {};
    std::vector<void*> allocs;
    uint64_t dev_bytes = 0;

    std::vector<LayerBufs> layers;
    bool io_loaded = false;
    float *cond_w0 = nullptr, *cond_w1 = nullptr, *cond_w2 = nullptr;
    float *in_w = nullptr, *in_b = nullptr, *out_norm_w = nullptr, *out_w = nullptr,
          *out_b = nullptr;
    int t_ctx = -1;

    // work buffers
    float* x = nullptr;   // [rows*S, D]
    void* h = nullptr;    // [rows*S, D]
    void* q = nullptr;    // [rows, H, S, Dh]
    void* ks = nullptr;
    void* vs = nullptr;   // V^T [rows, H, Dh, S'] (S' = S rounded up to 64), keys permuted
    void* gate = nullptr;  // [rows*S, D]
    void* o = nullptr;     // [rows*S, D]
    void* u = nullptr;     // [rows*S, F]
    // fp8 compute: the GEMM inputs h, o and u as e4m3 codes with E8M0 scales per 32 values.
    uint8_t *h8 = nullptr, *h8s = nullptr;  // [rows*S, D], [rows*S, D/32]
    uint8_t *o8 = nullptr, *o8s = nullptr;  // [rows*S, D], [rows*S, D/32]
    uint8_t *u8 = nullptr, *u8s = nullptr;  // [rows*S, F], [rows*S, F/32]
    // Fused adaLN (bf16 compute; GemmArgs): h holds x (1 + scale) of the next norm and rstat
    // the row sums of x^2 per 32 columns; the QKV+gate and W1|W3 GEMMs apply 1 / rms and add
    // the shift's product with their weights, biasq / bias13 [L][nvec_cap][N] per modulation
    // vector (computed with the table from the bf16 shift rows in shift_stage).
    bool fused = false;
    float* rstat = nullptr;     // [rows*S, D/32]
    float* biasq = nullptr;     // [L][nvec_cap][4D]
    float* bias13 = nullptr;    // [L][nvec_cap][2F], W1/W3 columns interleaved per 32
    void* shift_stage = nullptr;  // bf16 [2L][nvec_cap][D]
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    float* rope_cs = nullptr;  // [S, Dh/2, 2] interleaved (cos, sin), the QKVG epilogue's form
    float* xt = nullptr;    // [rows, S, P] sampler state / forward input
    float* vout = nullptr;  // [rows, S, P] head outputs (role-major in the sampler)
    float* xin = nullptr;   // [rows, S, P] Heun predictor state
    float* hist = nullptr;  // [4][rows, S, P] Heun v1 / PLMS-4 history
    RfEval* plan = nullptr; // sampler evaluations [2 * steps]
    int plan_cap = 0;       // steps
    // Context KV build on the device: projection input dims (0 text, 1 aux; 0 = absent),
    // their 64-padded widths, and a staging buffer for the states in the compute dtype.
    int ctx_dim[2] = {0, 0};
    int ctx_kpad[2] = {0, 0};
    void* ctx_state = nullptr;
    size_t ctx_state_bytes = 0;
    // Speaker-KV scaling (kv_scaling.rs:10-60): per-layer copies of the context K / V^T
    // with the aux keys of the scaled rows multiplied; the attention of layers < kvs_layers
    // reads them while kvs_on.
    std::vector<void*> act_k, act_v;
    bool kvs_on = false;
    int kvs_layers = 0;
    int* step = nullptr;    // device step counter; step[1]: the output head's finished-workgroup count
    int* zero_step = nullptr;
    // Latent key mask of the current call (build_joint_mask's self part,
    // attention.rs:730-750): per row and 64-key tile a validity word (bf16 attention)
    // and the float mask (f32 attention).  lat_on routes them to the attention launches.
    unsigned long long* lat_bits = nullptr;  // [rows, ceil(S / 64)] for the call's S
    float* lat_mask_f = nullptr;             // [rows, S]
    bool lat_on = false;

    // conditioning precompute
    int nvec_cap = 0;
    float* tvec = nullptr;
    float* emb = nullptr;
    float* h0 = nullptr;
    float* h1 = nullptr;
    float* cond = nullptr;
    float* mid = nullptr;
    float* tab = nullptr;
    VecLinJob* d_jobs_mlp = nullptr;   // 3 jobs
    VecLinJob* d_jobs_down = nullptr;  // L*6 jobs
    VecLinJob* d_jobs_up = nullptr;    // L*6 jobs

    GraphCache graphs;
};

namespace {

int dev_alloc(irodori_ctx* c, void** p, size_t bytes) { return tracked_alloc(c->allocs, c->dev_bytes, p, bytes); }

template <typename P>
int dalloc(irodori_ctx* c, P** p, size_t bytes) {
    return dev_alloc(c, reinterpret_cast<void**>(p), bytes);
}

// Key order of the V^T copies (latent and context): the 32x32x16 attention's for bf16 /
// fp8 contexts with 64-dim heads, the 16x16 attention's otherwise (f32, 128-dim heads).
bool vt_bf16_order(const irodori_ctx* c) { return c->bf16 && c->cfg.head_dim == 64; }

// Columns of the output head's W' rows for a P-channel latent (zeros past P).
int head_width(int P) { return P <= 32 ? 32 : P <= 64 ? 64 : P <= 128 ? 128 : 256; }




int upload(irodori_ctx* c, void* dst, const void* src, size_t bytes) {
    IRO_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    return IRODORI_OK;
}

// Host f32 [K, N] -> device compute-dtype [N, K] at dst (row offset applied by caller).
// tiled: dst in the tile-major layout of GemmArgs::w_tiled (through a row-major copy).
int ingest_kmajor(irodori_ctx* c, const float* host, int K, int N, int mode, void* dst, bool tiled = false) {
    float* stage = nullptr;
    void* rows = nullptr;
    size_t bytes = sizeof(float) * (size_t)K * N;
    IRO_HIP_CHECK(hipMalloc(&stage, bytes));
    hipError_t e = tiled ? hipMalloc(&rows, c->esz * (size_t)K * N) : hipSuccess;
    if (e == hipSuccess) e = hipMemcpyAsync(stage, host, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        void* out = tiled ? rows : dst;
        if (c->bf16)
            launch_transpose<bf16>(stage, K, N, mode, static_cast<bf16*>(out), c->stream);
        else
            launch_transpose<float>(stage, K, N, mode, static_cast<float*>(out), c->stream);
        if (tiled) launch_tile_rows(rows, N, (int)(c->esz * K), dst, c->stream);
        e = hipGetLastError();
    }
    hipError_t e2 = hipStreamSynchronize(c->stream);
    (void)hipFree(stage);
    if (rows) (void)hipFree(rows);
    if (e == hipSuccess) e = e2;
    if (e != hipSuccess) {
        set_last_error(std::string("weight ingest: ") + hipGetErrorString(e));
        return IRODORI_ERR_HIP;
    }
    return IRODORI_OK;
}

// Host f32 [K, N] -> device e4m3 codes [N, K] (row n = output channel, transpose mode as
// ingest_kmajor) at dst_q, and the channel scales at dst_s.
int ingest_fp8(irodori_ctx* c, const float* host, int K, int N, int mode, uint8_t* dst_q, float* dst_s,
               bool tiled = false) {
    float *stage = nullptr, *kmaj = nullptr;
    uint8_t* rows = nullptr;
    const size_t bytes = sizeof(float) * (size_t)K * N;
    IRO_HIP_CHECK(hipMalloc(&stage, bytes));
    hipError_t e = hipMalloc(&kmaj, bytes);
    if (e == hipSuccess && tiled) e = hipMalloc(&rows, (size_t)K * N);
    if (e == hipSuccess) e = hipMemcpyAsync(stage, host, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        launch_transpose<float>(stage, K, N, mode, kmaj, c->stream);
        launch_quant_weight_rows(kmaj, N, K, tiled ? rows : dst_q, dst_s, c->stream);
        if (tiled) launch_tile_rows(rows, N, K, dst_q, c->stream);
        e = hipGetLastError();
    }
    hipError_t e2 = hipStreamSynchronize(c->stream);
    (void)hipFree(stage);
    if (kmaj) (void)hipFree(kmaj);
    if (rows) (void)hipFree(rows);
    if (e == hipSuccess) e = e2;
    if (e != hipSuccess) {
        set_last_error(std::string("fp8 weight ingest: ") + hipGetErrorString(e));
        return IRODORI_ERR_HIP;
    }
    return IRODORI_OK;
}

int ensure_nvec(irodori_ctx* c, int nvec) {
    if (nvec <= c->nvec_cap) return IRODORI_OK;
    const auto& g = c->cfg;
    int D = g.model_dim, L = g.num_layers, r = g.adaln_rank;
    int cap = nvec < 64 ? 64 : nvec;
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    IRO_TRY(dalloc(c, &c->tvec, sizeof(float) * cap));
    IRO_TRY(dalloc(c, &c->emb, sizeof(float) * (size_t)cap * g.timestep_embed_dim));
    IRO_TRY(dalloc(c, &c->h0, sizeof(float) * (size_t)cap * D));
    IRO_TRY(dalloc(c, &c->h1, sizeof(float) * (size_t)cap * D));
    IRO_TRY(dalloc(c, &c->cond, sizeof(float) * (size_t)cap * 3 * D));
    IRO_TRY(dalloc(c, &c->mid, sizeof(float) * (size_t)L * 6 * cap * r));
    IRO_TRY(dalloc(c, &c->tab, sizeof(float) * (size_t)cap * L * 6 * D));
    if (c->fused) {
        IRO_TRY(dalloc(c, &c->biasq, sizeof(float) * (size_t)L * cap * 4 * D));
        IRO_TRY(dalloc(c, &c->bias13, sizeof(float) * (size_t)L * cap * 2 * c->Fp));
        IRO_TRY(dev_alloc(c, &c->shift_stage, sizeof(bf16) * (size_t)2 * L * cap * D));
    }
    c->nvec_cap = cap;

    // Job tables (pointers depend on the buffers above).
    std::vector<VecLinJob> mlp(3), down(L * 6), up(L * 6);
    mlp[0] = {c->emb, c->cond_w0, nullptr, nullptr, c->h0, g.timestep_embed_dim, 0, D,
              g.timestep_embed_dim, D, 0, 1};
    mlp[1] = {c->h0, c->cond_w1, nullptr, nullptr, c->h1, D, 0, D, D, D, 0, 1};
    mlp[2] = {c->h1, c->cond_w2, nullptr, nullptr, c->cond, D, 0, 3 * D, D, 3 * D, 0, 0};
    for (int l = 0; l < L; l++)
        for (int k = 0; k < 2; k++)
            for (int ch = 0; ch < 3; ch++) {
                int j = (l * 2 + k) * 3 + ch;
                float* midj = c->mid + (size_t)j * cap * r;
                auto& lb = c->layers[l];
                down[j] = {c->cond + ch * D, lb.ada_down[k][ch], nullptr, nullptr, midj, 3 * D, 0, r,
                           D, r, 1, 0};
                up[j] = {midj, lb.ada_up[k][ch], lb.ada_up_b[k][ch], c->cond + ch * D,
                         c->tab + (size_t)(l * 6 + k * 3 + ch) * D, r, 3 * D, L * 6 * D, r, D, 0,
                         ch == 2 ? 2 : 0};
            }
    if (!c->d_jobs_mlp) {
        IRO_TRY(dalloc(c, &c->d_jobs_mlp, sizeof(VecLinJob) * 3));
        IRO_TRY(dalloc(c, &c->d_jobs_down, sizeof(VecLinJob) * L * 6));
        IRO_TRY(dalloc(c, &c->d_jobs_up, sizeof(VecLinJob) * L * 6));
    }
    IRO_HIP_CHECK(hipMemcpy(c->d_jobs_mlp, mlp.data(), sizeof(VecLinJob) * 3, hipMemcpyHostToDevice));
    IRO_HIP_CHECK(hipMemcpy(c->d_jobs_down, down.data(), sizeof(VecLinJob) * L * 6, hipMemcpyHostToDevice));
    IRO_HIP_CHECK(hipMemcpy(c->d_jobs_up, up.data(), sizeof(VecLinJob) * L * 6, hipMemcpyHostToDevice));
    // Cached graphs captured the old table pointers.
    c->graphs.clear();
    return IRODORI_OK;
}

// Modulation table for nvec timesteps already in c->tvec (or, when skip_mlp, for cond
// vectors already in c->cond): tab[v][l][k][ch][:].  With the fused adaLN also the shift
// biases of layers [l0, l1) (whose weights must be loaded; all layers by default):
// biasq[l][v] = shift_attn(v, l) W_qkvg, bias13[l][v] = shift_mlp(v, l) W13.
int enqueue_mod_table(irodori_ctx* c, int nvec, bool skip_mlp, int l0 = 0, int l1 = -1) {
    const auto& g = c->cfg;
    int D = g.model_dim, L = g.num_layers, r = g.adaln_rank;
    if (l1 < 0) l1 = L;
    if (!skip_mlp) {
        RoctxRange cond("cond_module");  // timestep embedding + conditioning MLP (dit/model.rs:298-302)
        {
            RoctxRange te("timestep_embed");
            launch_timestep_embedding(c->tvec, nvec, g.timestep_embed_dim, c->emb, c->stream);
        }
        for (int j = 0; j < 3; j++)
            launch_vec_linear(c->d_jobs_mlp + j, 1, nvec, j == 2 ? 3 * D : D, c->stream);
    }
    launch_vec_linear(c->d_jobs_down, L * 6, nvec, r, c->stream);
    launch_vec_linear(c->d_jobs_up, L * 6, nvec, D, c->stream);
    if (c->fused) {
        const int cap = c->nvec_cap, F = c->Fp;
        bf16* stage = static_cast<bf16*>(c->shift_stage);
        launch_shift_stage(c->tab, nvec, cap, L, D, stage, c->stream);
        for (int l = l0; l < l1; l++)
            for (int k = 0; k < 2; k++) {
                GemmArgs<bf16> ga{};
                ga.A = stage + (size_t)(l * 2 + k) * cap * D;
                ga.W = static_cast<const bf16*>(k == 0 ? c->layers[l].w_qkvg : c->layers[l].w13);
                ga.w_tiled = c->w_tiled;
                ga.M = nvec;
                ga.N = k == 0 ? 4 * D : 2 * F;
                ga.K = D;
                ga.S = nvec;
                ga.C = (k == 0 ? c->biasq : c->bias13) + (size_t)l * cap * ga.N;
                if (launch_gemm<bf16>(EPI_STORE, ga, c->stream)) {
                    set_last_error("shift bias gemm shape");
                    return IRODORI_ERR_SHAPE;
                }
            }
    }
    return check_launch("modulation table");
}

// Whether a forward over B rows with modulation table mt runs the fused adaLN: the bf16
// context supports it and every row maps to one modulation vector (a sampler evaluation,
// or a single-row forward).  Decided from (mt, B) alone, so in_proj and every block part
// of the same forward agree.
bool fused_for(const irodori_ctx* c, const ModTable& mt, int B) { return c->fused && mt.rows_per_vec >= B; }

// The kernels of one DiT block (diffusion.rs:62-105), in launch order.  The block's
// first adaLN (attention modulation) is launched by the previous block's PART_NORM_NEXT
// or by in_proj.
enum LayerPart {
    PART_QKVG = 0,       // QKV + gate projection, head norms, half RoPE, V^T
    PART_ATTN = 1,       // joint attention + output gate
    PART_WO = 2,         // x += g_attn * (o @ W_o)
    PART_NORM_MLP = 3,   // mlp adaLN
    PART_W13 = 4,        // SwiGLU up-projection
    PART_W2 = 5,         // x += g_mlp * (m @ W2)
    PART_NORM_NEXT = 6,  // next block's attention adaLN (none after the last block)
    PART_COUNT = 7
};

// Options of one block part: the residual stream in a caller buffer instead of the
// context's (already offset to the slice's first row), and no next-norm operand from the
// W2 epilogue (an isolated MLP half).
struct PartOpts {
    float* x = nullptr;
    bool no_next = false;
};

// One kernel of a DiT block over batch rows [r0, r0 + B) of the context's buffers, on
// stream st.  Every row-indexed buffer is offset to row r0; mt must map the slice's local
// row b to the vector of global row r0 + b (rows_per_vec == 1 with the table offset, or
// all rows sharing one vector).
template <typename T>
int enqueue_part(irodori_ctx* c, int l, int B, int S, const ModTable& mt, int part, int r0,
                 hipStream_t st, const PartOpts& opt = PartOpts()) {
    const auto& g = c->cfg;
    const int D = g.model_dim, H = g.num_heads, F = c->Fp, M = B * S, Dh = g.head_dim;
    const bool last = l + 1 == g.num_layers;
    auto& lb = c->layers[l];
    const int vt_stride = (S + 63) / 64 * 64;
    const size_t tok0 = (size_t)r0 * S;  // first token row of the slice
    T* h = static_cast<T*>(c->h) + tok0 * D;
    float* x = opt.x ? opt.x : c->x + tok0 * D;
    T* q = static_cast<T*>(c->q) + (size_t)r0 * H * S * Dh;
    T* ks = static_cast<T*>(c->ks) + (size_t)r0 * H * S * Dh;
    T* vs = static_cast<T*>(c->vs) + (size_t)r0 * H * Dh * vt_stride;
    T* gate = static_cast<T*>(c->gate) + tok0 * D;
    T* o = static_cast<T*>(c->o) + tok0 * D;
    T* u = static_cast<T*>(c->u) + tok0 * F;
    // fp8 compute: the e4m3 copies of h / o / u with their block scales (same row slice).
    const bool f8 = c->fp8 && std::is_same<T, bf16>::value;
    // Fused adaLN (bf16): the partial sums of the slice's rows and this layer's shift biases.
    const bool fz = std::is_same<T, bf16>::value && fused_for(c, mt, B);
    float* rstat = fz ? c->rstat + tok0 * (D / 32) : nullptr;
    uint8_t* h8 = f8 ? c->h8 + tok0 * D : nullptr;
    uint8_t* h8s = f8 ? c->h8s + tok0 * (D / 32) : nullptr;
    uint8_t* o8 = f8 ? c->o8 + tok0 * D : nullptr;
    uint8_t* o8s = f8 ? c->o8s + tok0 * (D / 32) : nullptr;
    uint8_t* u8 = f8 ? c->u8 + tok0 * F : nullptr;
    uint8_t* u8s = f8 ? c->u8s + tok0 * (F / 32) : nullptr;
    // One projection: the bf16 / f32 GEMM on A and W, or the fp8 GEMM on their e4m3 forms
    // (block weights, tile-major when the context stores them so).
    auto gemm = [&](int epi, GemmArgs<T>& args, const T* A, const uint8_t* A8, const uint8_t* As,
                    const void* W, const float* ws) -> int {
        args.w_tiled = c->w_tiled;
        if constexpr (std::is_same<T, bf16>::value) {
            if (f8) {
                args.A8 = A8;
                args.As = As;
                args.W8 = static_cast<const uint8_t*>(W);
                args.ws = ws;
                return launch_gemm_fp8(epi, args, st);
            }
        }
        args.A = A;
        args.W = static_cast<const T*>(W);
        return launch_gemm<T>(epi, args, st);
    };

    GemmArgs<T> ga{};
    ga.mt = mt;
    ga.S = S;
    ga.layer = l;
    ga.H = H;
    ga.D = D;
    ga.eps = g.norm_eps;
    ga.M = M;
    ga.x = x;

    switch (part) {
        case PART_QKVG: {
            // QKV + gate projection with head norms and half RoPE (attention.rs:293-345, :423).
            ga.N = 4 * D;
            ga.K = D;
            ga.Q = q;
            ga.Kd = ks;
            ga.Vd = vs;
            ga.G = gate;
            ga.q_norm = lb.q_norm;
            ga.k_norm = lb.k_norm;
            ga.rope_cos = c->rope_cos;
            ga.rope_sin = c->rope_sin;
            ga.rope_cs = c->rope_cs;
            ga.vt_stride = vt_stride;
            ga.q_scale = 1.4426950408889634f / sqrtf((float)g.head_dim);
            if (fz) {
                ga.rstat = rstat;
                ga.rbias = c->biasq + (size_t)l * c->nvec_cap * 4 * D;
            }
            if (gemm(EPI_QKVG, ga, h, h8, h8s, lb.w_qkvg, lb.ws_qkvg)) {
                set_last_error("qkvg gemm shape");
                return IRODORI_ERR_SHAPE;
            }
            break;
        }
        case PART_ATTN: {
            // Joint attention over [latent self | cached ctx] (attention.rs:349-425).
            AttnArgs<T> aa{};
            aa.Q = q;
            aa.K0 = ks;
            aa.V0 = vs;
            aa.len0 = S;
            aa.stride0 = S;
            aa.v_transposed = true;
            aa.prescaled = true;
            aa.vstride0 = vt_stride;
            if (c->t_ctx > 0) {
                const int T1 = g.max_ctx, vs1 = (g.max_ctx + 63) / 64 * 64, nt1 = (g.max_ctx + 63) / 64;
                const bool kvs = c->kvs_on && l < c->kvs_layers;
                const T* ck = static_cast<const T*>(kvs ? c->act_k[l] : lb.ctx_k);
                const T* cv = static_cast<const T*>(kvs ? c->act_v[l] : lb.ctx_v);
                aa.K1 = ck + (size_t)r0 * H * T1 * Dh;
                aa.V1 = cv + (size_t)r0 * H * Dh * vs1;
                aa.len1 = c->t_ctx;
                aa.stride1 = T1;
                aa.vstride1 = vs1;
                aa.mask1 = lb.ctx_mask + (size_t)r0 * T1;
                aa.tile_on1 = lb.tile_on + (size_t)r0 * nt1;
                aa.bits1 = lb.tile_bits + (size_t)r0 * nt1;
            }
            if (c->lat_on) {
                aa.mask0 = c->lat_mask_f + tok0;
                aa.bits0 = c->lat_bits + (size_t)r0 * ((S + 63) / 64);
            }
            aa.B = B;
            aa.H = H;
            aa.Sq = S;
            aa.scale = 1.0f / sqrtf((float)g.head_dim);
            aa.out_mode = f8 ? 2 : 0;  // fp8: o goes straight to the W_o operand form
            aa.G = gate;
            aa.O = o;
            aa.O8 = o8;
            aa.O8s = o8s;
            int arc;
            if (Dh == 128)
                arc = launch_attention<T, 128>(aa, st);
            else if constexpr (std::is_same<T, bf16>::value)
                arc = launch_attention32(aa, st);
            else
                arc = launch_attention<T, 64>(aa, st);
            if (arc) { set_last_error("attention launch rejected the shape"); return IRODORI_ERR_SHAPE; }
            break;
        }
        case PART_WO: {
            // x += g_attn * (o @ Wo) (attention.rs:424, diffusion.rs:98).
            ga.N = D;
            ga.K = D;
            ga.kind = 0;
            if (fz) {  // and the mlp adaLN operand of this layer
                ga.Hn = h;
                ga.rstat_out = rstat;
                ga.next_layer = l;
                ga.next_kind = 1;
            }
            if (gemm(EPI_RESID, ga, o, o8, o8s, lb.w_o, lb.ws_o)) {
                set_last_error("wo gemm shape");
                return IRODORI_ERR_SHAPE;
            }
            break;
        }
        case PART_NORM_MLP: {
            // h2 = mlp adaLN(x) (diffusion.rs:101-102); fused into W_o / W13 with the fused adaLN.
            if (!fz) launch_norm_mod<T>(x, f8 ? nullptr : h, M, S, D, g.norm_eps, mt, l, 1, st, h8, h8s);
            break;
        }
        case PART_W13: {
            // m = silu(h2 W1) * (h2 W3) (feed_forward.rs:76-84).
            ga.N = 2 * F;
            ga.K = D;
            ga.U = u;
            ga.U8 = u8;  // fp8: m goes straight to the W2 operand form
            ga.U8s = u8s;
            if (fz) {
                ga.rstat = rstat;
                ga.rbias = c->bias13 + (size_t)l * c->nvec_cap * 2 * F;
            }
            if (gemm(EPI_SWIGLU, ga, h, h8, h8s, lb.w13, lb.ws_13)) {
                set_last_error("w13 gemm shape");
                return IRODORI_ERR_SHAPE;
            }
            break;
        }
        case PART_W2: {
            // x += g_mlp * (m @ W2) (diffusion.rs:104).
            ga.N = D;
            ga.K = F;
            ga.kind = 1;
            if (fz && !last && !opt.no_next) {  // and the next block's attention adaLN operand
                ga.Hn = h;
                ga.rstat_out = rstat;
                ga.next_layer = l + 1;
                ga.next_kind = 0;
            }
            if (gemm(EPI_RESID, ga, u, u8, u8s, lb.w2, lb.ws_2)) {
                set_last_error("w2 gemm shape");
                return IRODORI_ERR_SHAPE;
            }
            break;
        }
        case PART_NORM_NEXT: {
            // Next block's attention adaLN (fused into W2 / QKVG with the fused adaLN).
            if (!last && !fz && !opt.no_next) {
                launch_norm_mod<T>(x, f8 ? nullptr : h, M, S, D, g.norm_eps, mt, l + 1, 0, st, h8, h8s);
            }
            break;
        }
        default:
            set_last_error("unknown layer part");
            return IRODORI_ERR_INVALID_ARG;
    }
    return IRODORI_OK;
}

// One DiT block over batch rows [r0, r0 + B) on stream st (see enqueue_part).
template <typename T>
int enqueue_layer(irodori_ctx* c, int l, int B, int S, const ModTable& mt, int r0, hipStream_t st) {
    char name[32];
    snprintf(name, sizeof(name), "dit_block_%d", l);
    RoctxRange block(name);  // the reference's per-block and per-half ranges (diffusion.rs:88-104)
    {
        RoctxRange range("joint_attention_fused");
        for (int p : {PART_QKVG, PART_ATTN, PART_WO}) IRO_TRY(enqueue_part<T>(c, l, B, S, mt, p, r0, st));
    }
    {
        RoctxRange range("adaln_mlp");
        IRO_TRY(enqueue_part<T>(c, l, B, S, mt, PART_NORM_MLP, r0, st));
    }
    {
        RoctxRange range("swiglu_mlp_fused");
        for (int p : {PART_W13, PART_W2}) IRO_TRY(enqueue_part<T>(c, l, B, S, mt, p, r0, st));
    }
    {
        RoctxRange range("adaln_attn");  // the next block's attention adaLN, from this block's output
        IRO_TRY(enqueue_part<T>(c, l, B, S, mt, PART_NORM_NEXT, r0, st));
    }
    return check_launch("layer");
}

int enqueue_layer_any(irodori_ctx* c, int l, int B, int S, const ModTable& mt, int r0 = 0,
                      hipStream_t st = nullptr) {
    if (!st) st = c->stream;
    return c->bf16 ? enqueue_layer<bf16>(c, l, B, S, mt, r0, st) : enqueue_layer<float>(c, l, B, S, mt, r0, st);
}

// in_proj + the first adaLN for batch rows [r0, r0 + B): row r0 + b reads source row
// b mod src_batches of src [src_batches, S, P].  When every row shares one modulation vector
// (a sampler evaluation's roles), the src_batches distinct rows are computed once and
// written B / src_batches times.
int enqueue_inproj(irodori_ctx* c, int B, int S, const float* src, int src_batches, int r0, const ModTable& mt,
                   hipStream_t st) {
    const auto& g = c->cfg;
    const size_t tok0 = (size_t)r0 * S;
    float* x = c->x + tok0 * g.model_dim;
    const bool rep = B > src_batches && B % src_batches == 0 && mt.rows_per_vec >= B;
    const int copies = rep ? B / src_batches : 1, Bc = B / copies;
    if (c->bf16) {
        bf16* h = c->fp8 ? nullptr : static_cast<bf16*>(c->h) + tok0 * g.model_dim;
        launch_inproj_norm<bf16>(src, src_batches, c->in_w, c->in_b, x, h, Bc * S, S, g.latent_dim, g.model_dim,
                                 g.norm_eps, mt, st, c->fp8 ? c->h8 + tok0 * g.model_dim : nullptr,
                                 c->fp8 ? c->h8s + tok0 * (g.model_dim / 32) : nullptr,
                                 fused_for(c, mt, B) ? c->rstat + tok0 * (g.model_dim / 32) : nullptr, copies);
    }
    else
        launch_inproj_norm<float>(src, src_batches, c->in_w, c->in_b, x,
                                  static_cast<float*>(c->h) + tok0 * g.model_dim, Bc * S, S, g.latent_dim,
                                  g.model_dim, g.norm_eps, mt, st, nullptr, nullptr, nullptr, copies);
    return check_launch("in_proj");
}

// Output head for batch rows [r0, r0 + B) into the matching rows of vout.
int enqueue_head(irodori_ctx* c, int B, int S, int r0, hipStream_t st) {
    const auto& g = c->cfg;
    FinalArgs fa{};
    fa.x = c->x + (size_t)r0 * S * g.model_dim;
    fa.norm_w = c->out_norm_w;
    fa.out_w = c->out_w;
    fa.out_b = c->out_b;
    fa.B = B;
    fa.S = S;
    fa.D = g.model_dim;
    fa.P = g.latent_dim;
    fa.eps = g.norm_eps;
    fa.v_out = c->vout + (size_t)r0 * S * g.latent_dim;
    launch_final(fa, st);
    return check_launch("output head");
}

// All kernels of one sampler evaluation (one model forward per active role, then the
// update): every active role r runs in_proj from src and the L blocks over its rows
// [r U, r U + U) as an independent chain of kernels — the first on the context's stream,
// the others on side streams forked from it and joined before the output head, which
// computes every active role's velocity and applies the guided combine and the integrator
// update in one kernel.  Rows never interact inside the forward, so in a captured graph the chains
// overlap each other's launch gaps, tails and uneven attention work (the conditioned
// role attends to the context, a dropped signal's keys are skipped).  Every row shares
// the evaluation's modulation vector (mt.step_add selects t_{i+1} for the Heun
// corrector).  The step counter advances after the step's last evaluation.
int enqueue_eval(irodori_ctx* c, int U, int S, int roles, int method, int phase, const float* src) {
    const auto& g = c->cfg;
    // Every row of the evaluation (b < kMaxRoles U, chain-local or not) maps to vector step.
    ModTable mt{c->tab, c->step, 1, U * irodori_ctx::kMaxRoles, g.num_layers, phase};
    int active[irodori_ctx::kMaxRoles], na = 0;
    for (int r = 0; r < irodori_ctx::kMaxRoles; r++)
        if (roles & (1 << r)) active[na++] = r;
    if (na == 0) { set_last_error("no role to evaluate"); return IRODORI_ERR_INVALID_ARG; }
    // in_proj of every active row in one launch before the fork when the active roles are
    // the first na (rows [0, na U)), else at the head of each chain.
    const bool contiguous = active[na - 1] == na - 1;
    if (contiguous) IRO_TRY(enqueue_inproj(c, na * U, S, src, U, 0, mt, c->stream));
    if (na > 1) IRO_HIP_CHECK(hipEventRecord(c->ev_fork, c->stream));
    // The chains are captured last role first: the first role (the conditioned one, whose
    // attention also reads the context) is then captured last, which measured 0.07-0.2 ms
    // faster per 40-step run at config 4 than the opposite order (never slower in 5 pairs).
    for (int kk = 0; kk < na; kk++) {
        const int k = na - 1 - kk;
        hipStream_t st = k == 0 ? c->stream : c->side[k - 1];
        if (k > 0) IRO_HIP_CHECK(hipStreamWaitEvent(st, c->ev_fork, 0));
        const int r0 = active[k] * U;
        if (!contiguous) IRO_TRY(enqueue_inproj(c, U, S, src, U, r0, mt, st));
        for (int l = 0; l < g.num_layers; l++) IRO_TRY(enqueue_layer_any(c, l, U, S, mt, r0, st));
        if (k > 0) IRO_HIP_CHECK(hipEventRecord(c->ev_join[k - 1], st));
    }
    for (int k = 1; k < na; k++) IRO_HIP_CHECK(hipStreamWaitEvent(c->stream, c->ev_join[k - 1], 0));
    FinalArgs fa{};
    fa.x = c->x;
    fa.norm_w = c->out_norm_w;
    fa.out_w = c->out_w;
    fa.out_b = c->out_b;
    fa.B = U;
    fa.S = S;
    fa.D = g.model_dim;
    fa.P = g.latent_dim;
    fa.eps = g.norm_eps;
    fa.nrole = na;
    for (int k = 0; k < na; k++) fa.role[k] = active[k];
    fa.rf.x = c->xt;
    fa.rf.xin = c->xin;
    fa.rf.hist = c->hist;
    fa.rf.plan = c->plan;
    fa.rf.step = c->step;
    fa.rf.done = c->step + 1;
    fa.rf.advance = method != IRODORI_METHOD_HEUN || phase == 1;
    fa.rf.phase = phase;
    fa.rf.method = method;
    fa.rf.n = U * S * g.latent_dim;
    launch_final(fa, c->stream);
    return check_launch("sampler evaluation");
}

int check_ready(irodori_ctx* c, int B) {
    IRO_REQUIRE(c->io_loaded, IRODORI_ERR_NOT_LOADED, "io weights not loaded");
    for (int l = 0; l < c->cfg.num_layers; l++) {
        IRO_REQUIRE(c->layers[l].loaded, IRODORI_ERR_NOT_LOADED,
                    "block weights of layer " + std::to_string(l) + " not loaded");
        if (c->t_ctx > 0)
            for (int r = 0; r < B; r++)
                IRO_REQUIRE(c->layers[l].row_set[r], IRODORI_ERR_NOT_LOADED,
                            "context KV of layer " + std::to_string(l) + " row " + std::to_string(r) +
                                " not set");
    }
    return IRODORI_OK;
}

// Active CFG signals in the sampler's order (euler_sampler.rs:163-200): text if its scale
// is > 0, speaker if the condition holds a speaker state and its scale is > 0, caption if
// the condition holds a caption with a valid token and its scale is > 0.  scales[k] = the
// k-th active signal's scale; returns the count.
int cfg_signals(const irodori_sampler_params* p, float* scales) {
    int n = 0;
    if (p->scale_text > 0.f) scales[n++] = p->scale_text;
    if (p->has_speaker && p->scale_speaker > 0.f) scales[n++] = p->scale_speaker;
    if (p->has_caption && p->scale_caption > 0.f) scales[n++] = p->scale_caption;
    return n;
}

int validate_params(const irodori_sampler_params* p) {
    IRO_REQUIRE(p != nullptr, IRODORI_ERR_INVALID_ARG, "params is null");
    IRO_REQUIRE(p->num_steps > 0, IRODORI_ERR_CONFIG, "num_steps must be > 0");
    const char* names[3] = {"guidance.scale_text", "guidance.scale_caption", "guidance.scale_speaker"};
    float sc[3] = {p->scale_text, p->scale_caption, p->scale_speaker};
    for (int i = 0; i < 3; i++)
        IRO_REQUIRE(std::isfinite(sc[i]), IRODORI_ERR_CONFIG,
                    std::string(names[i]) + " must be finite, got " + std::to_string(sc[i]));
    IRO_REQUIRE(std::isfinite(p->min_t) && p->min_t >= 0.f && p->min_t <= 1.f, IRODORI_ERR_CONFIG,
                "guidance.min_t must be finite and in [0, 1], got " + std::to_string(p->min_t));
    IRO_REQUIRE(std::isfinite(p->max_t) && p->max_t >= 0.f && p->max_t <= 1.f, IRODORI_ERR_CONFIG,
                "guidance.max_t must be finite and in [0, 1], got " + std::to_string(p->max_t));
    IRO_REQUIRE(p->min_t <= p->max_t, IRODORI_ERR_CONFIG,
                "guidance.min_t (" + std::to_string(p->min_t) + ") must not exceed guidance.max_t (" +
                    std::to_string(p->max_t) + ")");
    IRO_REQUIRE(!p->has_truncation || (std::isfinite(p->truncation_factor) && p->truncation_factor > 0.f),
                IRODORI_ERR_CONFIG, "truncation_factor must be finite and > 0");
    IRO_REQUIRE(!(p->method == IRODORI_METHOD_PLMS4 && p->cfg_mode == IRODORI_CFG_ALTERNATING),
                IRODORI_ERR_CONFIG,
                "sampler PLMS4 is not compatible with cfg_guidance_mode=Alternating; use Independent or "
                "Joint instead");
    IRO_REQUIRE(p->method >= 0 && p->method <= 2, IRODORI_ERR_CONFIG, "unknown sampler method");
    // The condition's auxiliary state is a speaker or a caption, never both
    // (AuxConditioner, aux_conditioner.rs:43-52).
    IRO_REQUIRE(!(p->has_speaker && p->has_caption), IRODORI_ERR_CONFIG,
                "has_speaker and has_caption are exclusive: the auxiliary condition is a speaker or a caption");
    IRO_REQUIRE(p->cfg_mode >= 0 && p->cfg_mode <= 2, IRODORI_ERR_CONFIG, "unknown cfg guidance mode");
    if (p->has_temporal_rescale) {
        IRO_REQUIRE(std::isfinite(p->rescale_k), IRODORI_ERR_CONFIG, "temporal_rescale.k must be finite");
        IRO_REQUIRE(p->rescale_sigma != 0.f, IRODORI_ERR_CONFIG, "temporal_rescale.sigma must not be zero");
    }
    if (p->has_speaker_kv) {
        IRO_REQUIRE(std::isfinite(p->speaker_kv_scale) && p->speaker_kv_scale > 0.f, IRODORI_ERR_CONFIG,
                    "speaker_kv.scale must be finite and > 0");
        IRO_REQUIRE(!p->speaker_kv_has_min_t ||
                        (std::isfinite(p->speaker_kv_min_t) && p->speaker_kv_min_t >= 0.f && p->speaker_kv_min_t <= 1.f),
                    IRODORI_ERR_CONFIG, "speaker_kv.min_t must be finite and in [0, 1]");
    }
    if (p->cfg_mode == IRODORI_CFG_JOINT) {
        // euler_sampler.rs:209-228: all active scales must match.
        float act[3];
        const int n = cfg_signals(p, act);
        float lo = INFINITY, hi = -INFINITY;
        for (int k = 0; k < n; k++) { lo = fminf(lo, act[k]); hi = fmaxf(hi, act[k]); }
        IRO_REQUIRE(!(hi - lo >= 1e-6f), IRODORI_ERR_CONFIG,
                    "cfg_guidance_mode=Joint requires all active cfg scales to be equal, but got text=" +
                        std::to_string(p->scale_text) + ", speaker=" + std::to_string(p->scale_speaker) +
                        ", caption=" + std::to_string(p->scale_caption));
    }
    return IRODORI_OK;
}

// Number of sampler roles (context bundles) for n active signals (role-major rows).
int cfg_roles(const irodori_sampler_params* p, int n) {
    return p->cfg_mode == IRODORI_CFG_JOINT ? (n > 0 ? 2 : 1) : 1 + n;
}

}  // namespace


extern "C" {

const char* irodori_last_error(void) { return g_last_error.c_str(); }
const char* irodori_version(void) { return "irodori_hip 0.1.0 (gfx950)"; }

int irodori_sampler_params_validate(const irodori_sampler_params* params) {
    IRO_GUARD_BEGIN
    return validate_params(params);
    IRO_GUARD_END
}

int irodori_ctx_destroy(irodori_ctx* c) {
    if (!c) return IRODORI_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    c->graphs.clear();
    for (void* p : c->allocs) (void)hipFree(p);
    for (auto sd : c->side)
        if (sd) (void)hipStreamSynchronize(sd);
    if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
    for (auto ev : c->ev_join)
        if (ev) (void)hipEventDestroy(ev);
    for (auto sd : c->side)
        if (sd) (void)hipStreamDestroy(sd);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return IRODORI_OK;
}

int irodori_ctx_create(int device, const irodori_dit_config* cfg, irodori_ctx** out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(cfg && out, IRODORI_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    const irodori_dit_config& g = *cfg;
    IRO_REQUIRE(g.compute_dtype == IRODORI_DTYPE_BF16 || g.compute_dtype == IRODORI_DTYPE_F32 ||
                    g.compute_dtype == IRODORI_DTYPE_FP8,
                IRODORI_ERR_DTYPE, "compute_dtype must be IRODORI_DTYPE_BF16, _F32 or _FP8");
    IRO_REQUIRE(g.compute_dtype != IRODORI_DTYPE_FP8 || g.model_dim % 128 == 0, IRODORI_ERR_SHAPE,
                "fp8 compute needs a model_dim multiple of 128");
    IRO_REQUIRE(g.num_layers > 0 && g.num_heads > 0 && g.model_dim > 0 && g.latent_dim > 0,
                IRODORI_ERR_SHAPE, "dimensions must be positive");
    IRO_REQUIRE(g.head_dim == 64 || g.head_dim == 128, IRODORI_ERR_SHAPE, "head_dim must be 64 or 128");
    IRO_REQUIRE(g.compute_dtype != IRODORI_DTYPE_FP8 || g.head_dim == 64, IRODORI_ERR_SHAPE,
                "fp8 compute needs head_dim 64");
    IRO_REQUIRE(g.num_heads * g.head_dim == g.model_dim, IRODORI_ERR_SHAPE, "num_heads * head_dim must equal model_dim");
    IRO_REQUIRE(g.model_dim % 64 == 0 && g.model_dim <= 4096, IRODORI_ERR_SHAPE,
                "model_dim must be a multiple of 64 and <= 4096");
    IRO_REQUIRE(g.mlp_hidden > 0, IRODORI_ERR_SHAPE, "mlp_hidden must be positive");
    IRO_REQUIRE(g.latent_dim <= 256, IRODORI_ERR_SHAPE, "latent_dim (patched) must be <= 256");
    IRO_REQUIRE(g.adaln_rank > 0 && g.timestep_embed_dim > 0 && g.timestep_embed_dim % 2 == 0,
                IRODORI_ERR_SHAPE, "adaln_rank > 0 and even timestep_embed_dim required");
    IRO_REQUIRE(g.norm_eps > 0.f && std::isfinite(g.norm_eps), IRODORI_ERR_CONFIG, "norm_eps must be > 0");
    IRO_REQUIRE(g.max_rows > 0 && g.max_seq > 0 && g.max_ctx >= 0, IRODORI_ERR_SHAPE, "max sizes must be positive");
    IRO_REQUIRE(g.max_rows <= 65535, IRODORI_ERR_SHAPE, "max_rows must be <= 65535 (one output-head grid row per group)");
    // The 16-bit joint attention lists a row's key tiles (latent, then context) in registers.
    IRO_REQUIRE(g.compute_dtype == IRODORI_DTYPE_F32 ||
                    (g.max_seq + 63) / 64 + (g.max_ctx + 63) / 64 <= kAttnMaxKeyTiles,
                IRODORI_ERR_SHAPE,
                "max_seq and max_ctx rounded up to 64 keys each must total at most " +
                    std::to_string(64 * kAttnMaxKeyTiles) + " keys (the bf16 / fp8 attention's key-tile list)");

    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    IRO_REQUIRE(e == hipSuccess && ndev > 0, IRODORI_ERR_HIP,
                std::string("no HIP device available: ") + (e == hipSuccess ? "0 devices" : hipGetErrorString(e)));
    IRO_REQUIRE(device >= 0 && device < ndev, IRODORI_ERR_INVALID_ARG, "device index out of range");
    IRO_HIP_CHECK(hipSetDevice(device));

    std::unique_ptr<irodori_ctx, int (*)(irodori_ctx*)> c(new irodori_ctx(), irodori_ctx_destroy);
    c->device = device;
    c->cfg = g;
    c->Fp = (g.mlp_hidden + 127) / 128 * 128;
    c->fp8 = g.compute_dtype == IRODORI_DTYPE_FP8;
    c->bf16 = g.compute_dtype == IRODORI_DTYPE_BF16 || c->fp8;
    c->esz = c->bf16 ? 2 : 4;
    c->w_tiled = !c->fp8 || (g.model_dim % 128 == 0 && (g.num_heads * g.head_dim) % 128 == 0);
    // The fused adaLN's GEMMs take the row partial sums as up to 16 float4 per row.
    c->fused = c->bf16 && !c->fp8 && g.model_dim % 128 == 0 && g.model_dim <= 2048;
    IRO_HIP_CHECK(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    IRO_HIP_CHECK(hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming));
    for (int i = 0; i < irodori_ctx::kMaxRoles - 1; i++) {
        IRO_HIP_CHECK(hipStreamCreateWithFlags(&c->side[i], hipStreamNonBlocking));
        IRO_HIP_CHECK(hipEventCreateWithFlags(&c->ev_join[i], hipEventDisableTiming));
    }

    int D = g.model_dim, F = c->Fp, H = g.num_heads, Dh = g.head_dim, L = g.num_layers;
    int R = g.max_rows, S = g.max_seq, T = g.max_ctx > 0 ? g.max_ctx : 1, P = g.latent_dim;
    size_t es = c->esz, M = (size_t)R * S;
    c->layers.resize(L);
    int ntl = (T + 63) / 64;
    int Tp = ntl * 64, Sp = (S + 63) / 64 * 64;
    for (int l = 0; l < L; l++) {
        auto& lb = c->layers[l];
        const size_t wes = c->fp8 ? 1 : es;  // weight element bytes
        IRO_TRY(dev_alloc(c.get(), &lb.w_qkvg, wes * 4 * D * D));
        IRO_TRY(dev_alloc(c.get(), &lb.w_o, wes * D * D));
        IRO_TRY(dev_alloc(c.get(), &lb.w13, wes * 2 * (size_t)F * D));
        IRO_TRY(dev_alloc(c.get(), &lb.w2, wes * (size_t)D * F));
        if (c->fp8) {
            IRO_TRY(dalloc(c.get(), &lb.ws_qkvg, sizeof(float) * 4 * D));
            IRO_TRY(dalloc(c.get(), &lb.ws_o, sizeof(float) * D));
            IRO_TRY(dalloc(c.get(), &lb.ws_13, sizeof(float) * 2 * F));
            IRO_TRY(dalloc(c.get(), &lb.ws_2, sizeof(float) * D));
        }
        IRO_TRY(dalloc(c.get(), &lb.q_norm, sizeof(float) * H * Dh));
        IRO_TRY(dalloc(c.get(), &lb.k_norm, sizeof(float) * H * Dh));
        for (int k = 0; k < 2; k++)
            for (int ch = 0; ch < 3; ch++) {
                IRO_TRY(dalloc(c.get(), &lb.ada_down[k][ch], sizeof(float) * (size_t)D * g.adaln_rank));
                IRO_TRY(dalloc(c.get(), &lb.ada_up[k][ch], sizeof(float) * (size_t)g.adaln_rank * D));
                IRO_TRY(dalloc(c.get(), &lb.ada_up_b[k][ch], sizeof(float) * D));
            }
        IRO_TRY(dev_alloc(c.get(), &lb.ctx_k, es * (size_t)R * H * T * Dh));
        IRO_TRY(dev_alloc(c.get(), &lb.ctx_v, es * (size_t)R * H * Dh * Tp));
        IRO_HIP_CHECK(hipMemsetAsync(lb.ctx_v, 0, es * (size_t)R * H * Dh * Tp, c->stream));
        IRO_TRY(dalloc(c.get(), &lb.ctx_mask, sizeof(float) * (size_t)R * T));
        IRO_TRY(dalloc(c.get(), &lb.tile_on, sizeof(int) * (size_t)R * ntl));
        IRO_TRY(dalloc(c.get(), &lb.tile_bits, sizeof(unsigned long long) * (size_t)R * ntl));
        lb.row_set.assign(R, 0);
    }
    IRO_TRY(dalloc(c.get(), &c->cond_w0, sizeof(float) * (size_t)g.timestep_embed_dim * D));
    IRO_TRY(dalloc(c.get(), &c->cond_w1, sizeof(float) * (size_t)D * D));
    IRO_TRY(dalloc(c.get(), &c->cond_w2, sizeof(float) * (size_t)D * 3 * D));
    IRO_TRY(dalloc(c.get(), &c->in_w, sizeof(float) * (size_t)P * D));
    IRO_TRY(dalloc(c.get(), &c->in_b, sizeof(float) * D));
    IRO_TRY(dalloc(c.get(), &c->out_norm_w, sizeof(float) * D));
    IRO_TRY(dalloc(c.get(), &c->out_w, sizeof(float) * (size_t)D * head_width(P)));
    IRO_TRY(dalloc(c.get(), &c->out_b, sizeof(float) * P));

    IRO_TRY(dalloc(c.get(), &c->x, sizeof(float) * M * D));
    IRO_TRY(dev_alloc(c.get(), &c->h, es * M * D));
    IRO_TRY(dev_alloc(c.get(), &c->q, es * M * D));
    IRO_TRY(dev_alloc(c.get(), &c->ks, es * M * D));
    IRO_TRY(dev_alloc(c.get(), &c->vs, es * (size_t)R * H * Dh * Sp));
    IRO_HIP_CHECK(hipMemsetAsync(c->vs, 0, es * (size_t)R * H * Dh * Sp, c->stream));
    IRO_TRY(dev_alloc(c.get(), &c->gate, es * M * D));
    IRO_TRY(dev_alloc(c.get(), &c->o, es * M * D));
    IRO_TRY(dev_alloc(c.get(), &c->u, es * M * F));
    if (c->fused) IRO_TRY(dalloc(c.get(), &c->rstat, sizeof(float) * M * (D / 32)));
    if (c->fp8) {
        IRO_TRY(dalloc(c.get(), &c->h8, M * D));
        IRO_TRY(dalloc(c.get(), &c->h8s, M * D / 32));
        IRO_TRY(dalloc(c.get(), &c->o8, M * D));
        IRO_TRY(dalloc(c.get(), &c->o8s, M * D / 32));
        IRO_TRY(dalloc(c.get(), &c->u8, M * F));
        IRO_TRY(dalloc(c.get(), &c->u8s, M * F / 32));
    }
    IRO_TRY(dalloc(c.get(), &c->rope_cos, sizeof(float) * (size_t)S * Dh / 2));
    IRO_TRY(dalloc(c.get(), &c->rope_sin, sizeof(float) * (size_t)S * Dh / 2));
    IRO_TRY(dalloc(c.get(), &c->rope_cs, sizeof(float) * (size_t)S * Dh));
    IRO_TRY(dalloc(c.get(), &c->xt, sizeof(float) * M * P));
    IRO_TRY(dalloc(c.get(), &c->vout, sizeof(float) * M * P));
    IRO_TRY(dalloc(c.get(), &c->xin, sizeof(float) * M * P));
    IRO_TRY(dalloc(c.get(), &c->hist, sizeof(float) * 4 * M * P));
    IRO_TRY(dalloc(c.get(), &c->lat_bits, sizeof(unsigned long long) * (size_t)R * ((S + 63) / 64)));
    IRO_TRY(dalloc(c.get(), &c->lat_mask_f, sizeof(float) * (size_t)R * S));
    IRO_TRY(dalloc(c.get(), &c->step, 2 * sizeof(int)));
    IRO_TRY(dalloc(c.get(), &c->zero_step, sizeof(int)));
    IRO_HIP_CHECK(hipMemsetAsync(c->zero_step, 0, sizeof(int), c->stream));

    std::vector<float> cs, sn;
    host_rope_tables(S, Dh, g.rope_theta, cs, sn);
    IRO_TRY(upload(c.get(), c->rope_cos, cs.data(), sizeof(float) * cs.size()));
    IRO_TRY(upload(c.get(), c->rope_sin, sn.data(), sizeof(float) * sn.size()));
    std::vector<float> csi(cs.size() * 2);
    for (size_t i = 0; i < cs.size(); i++) {
        csi[2 * i] = cs[i];
        csi[2 * i + 1] = sn[i];
    }
    IRO_TRY(upload(c.get(), c->rope_cs, csi.data(), sizeof(float) * csi.size()));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    *out = c.release();
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_ctx_device_bytes(const irodori_ctx* c, uint64_t* bytes) {
    IRO_REQUIRE(c && bytes, IRODORI_ERR_INVALID_ARG, "null argument");
    *bytes = c->dev_bytes;
    return IRODORI_OK;
}

int irodori_load_io_weights(irodori_ctx* c, const irodori_io_weights* w) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && w, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(w->cond_w0 && w->cond_w1 && w->cond_w2 && w->in_w && w->in_b && w->out_norm_w &&
                    w->out_w && w->out_b,
                IRODORI_ERR_INVALID_ARG, "null io weight pointer");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const auto& g = c->cfg;
    int D = g.model_dim, P = g.latent_dim;
    IRO_TRY(upload(c, c->cond_w0, w->cond_w0, sizeof(float) * (size_t)g.timestep_embed_dim * D));
    IRO_TRY(upload(c, c->cond_w1, w->cond_w1, sizeof(float) * (size_t)D * D));
    IRO_TRY(upload(c, c->cond_w2, w->cond_w2, sizeof(float) * (size_t)D * 3 * D));
    IRO_TRY(upload(c, c->in_w, w->in_w, sizeof(float) * (size_t)P * D));
    IRO_TRY(upload(c, c->in_b, w->in_b, sizeof(float) * D));
    IRO_TRY(upload(c, c->out_norm_w, w->out_norm_w, sizeof(float) * D));
    // Output head weight with the out_norm weight folded in, rows padded to PW columns
    // (zeros past P) for the head's whole-row loads.
    const int PW = head_width(P);
    std::vector<float> wt((size_t)D * PW, 0.f);
    for (int d = 0; d < D; d++)
        for (int p = 0; p < P; p++) wt[(size_t)d * PW + p] = w->out_w[(size_t)d * P + p] * w->out_norm_w[d];
    IRO_TRY(upload(c, c->out_w, wt.data(), sizeof(float) * wt.size()));
    IRO_TRY(upload(c, c->out_b, w->out_b, sizeof(float) * P));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    c->io_loaded = true;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_load_block_weights(irodori_ctx* c, int layer, const irodori_block_weights* w) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && w, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(layer >= 0 && layer < c->cfg.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(w->w_qkv && w->w_gate && w->w_o && w->q_norm && w->k_norm && w->w13 && w->w2,
                IRODORI_ERR_INVALID_ARG, "null block weight pointer");
    for (int k = 0; k < 2; k++)
        for (int ch = 0; ch < 3; ch++)
            IRO_REQUIRE(w->ada_down[k][ch] && w->ada_up[k][ch] && w->ada_up_b[k][ch], IRODORI_ERR_INVALID_ARG,
                        "null adaLN weight pointer");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const auto& g = c->cfg;
    const int D = g.model_dim, F = g.mlp_hidden, Fp = c->Fp, HD = g.num_heads * g.head_dim, r = g.adaln_rank;
    // SwiGLU weights padded to Fp on the host: [W1 | 0 | W3 | 0] and W2 with zero rows.
    std::vector<float> w13p, w2p;
    const float* w13 = w->w13;
    const float* w2 = w->w2;
    if (Fp != F) {
        w13p.assign((size_t)D * 2 * Fp, 0.f);
        for (int d = 0; d < D; d++) {
            std::copy(w->w13 + (size_t)d * 2 * F, w->w13 + (size_t)d * 2 * F + F, w13p.data() + (size_t)d * 2 * Fp);
            std::copy(w->w13 + (size_t)d * 2 * F + F, w->w13 + (size_t)d * 2 * F + 2 * F,
                      w13p.data() + (size_t)d * 2 * Fp + Fp);
        }
        w2p.assign((size_t)Fp * D, 0.f);
        std::copy(w->w2, w->w2 + (size_t)F * D, w2p.data());
        w13 = w13p.data();
        w2 = w2p.data();
    }
    auto& lb = c->layers[layer];
    char* qkvg = static_cast<char*>(lb.w_qkvg);
    if (c->fp8) {
        uint8_t* q8 = reinterpret_cast<uint8_t*>(qkvg);
        // (The gate rows start a 64-row group: 3 H Dh is a multiple of 64.)
        const bool t = c->w_tiled;
        IRO_TRY(ingest_fp8(c, w->w_qkv, D, 3 * HD, 0, q8, lb.ws_qkvg, t));
        IRO_TRY(ingest_fp8(c, w->w_gate, D, D, 0, q8 + (size_t)3 * HD * D, lb.ws_qkvg + 3 * HD, t));
        IRO_TRY(ingest_fp8(c, w->w_o, HD, D, 0, static_cast<uint8_t*>(lb.w_o), lb.ws_o, t));
        IRO_TRY(ingest_fp8(c, w13, D, 2 * Fp, 1, static_cast<uint8_t*>(lb.w13), lb.ws_13, t));
        IRO_TRY(ingest_fp8(c, w2, Fp, D, 0, static_cast<uint8_t*>(lb.w2), lb.ws_2, t));
    } else {
        const bool t = c->w_tiled;
        IRO_TRY(ingest_kmajor(c, w->w_qkv, D, 3 * HD, 0, qkvg, t));
        IRO_TRY(ingest_kmajor(c, w->w_gate, D, D, 0, qkvg + c->esz * (size_t)3 * HD * D, t));
        IRO_TRY(ingest_kmajor(c, w->w_o, HD, D, 0, lb.w_o, t));
        IRO_TRY(ingest_kmajor(c, w13, D, 2 * Fp, 1, lb.w13, t));
        IRO_TRY(ingest_kmajor(c, w2, Fp, D, 0, lb.w2, t));
    }
    IRO_TRY(upload(c, lb.q_norm, w->q_norm, sizeof(float) * HD));
    IRO_TRY(upload(c, lb.k_norm, w->k_norm, sizeof(float) * HD));
    for (int k = 0; k < 2; k++)
        for (int ch = 0; ch < 3; ch++) {
            IRO_TRY(upload(c, lb.ada_down[k][ch], w->ada_down[k][ch], sizeof(float) * (size_t)D * r));
            IRO_TRY(upload(c, lb.ada_up[k][ch], w->ada_up[k][ch], sizeof(float) * (size_t)r * D));
            IRO_TRY(upload(c, lb.ada_up_b[k][ch], w->ada_up_b[k][ch], sizeof(float) * D));
        }
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    lb.loaded = true;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_clear_ctx_kv(irodori_ctx* c) {
    IRO_REQUIRE(c, IRODORI_ERR_INVALID_ARG, "null context");
    c->t_ctx = -1;
    for (auto& lb : c->layers) std::fill(lb.row_set.begin(), lb.row_set.end(), 0);
    c->graphs.clear();
    return IRODORI_OK;
}

// The context key mask of one row of one layer (nonzero = attend) as the attention reads
// it: a float mask [max_ctx], per-tile "any valid key" flags and 64-bit validity words.
static int upload_row_mask(irodori_ctx* c, LayerBufs& lb, int row, int t_ctx, const uint8_t* mask) {
    const int T = c->cfg.max_ctx > 0 ? c->cfg.max_ctx : 1;
    std::vector<float> m(T, 0.f);
    int ntl = (T + 63) / 64;
    std::vector<int> on(ntl, 0);
    std::vector<unsigned long long> bits(ntl, 0ull);
    for (int j = 0; j < t_ctx; j++) {
        m[j] = mask[j] ? 1.f : 0.f;
        if (mask[j]) {
            on[j / 64] = 1;
            bits[j / 64] |= 1ull << (j % 64);
        }
    }
    IRO_TRY(upload(c, lb.ctx_mask + (size_t)row * T, m.data(), sizeof(float) * T));
    IRO_TRY(upload(c, lb.tile_on + (size_t)row * ntl, on.data(), sizeof(int) * ntl));
    IRO_TRY(upload(c, lb.tile_bits + (size_t)row * ntl, bits.data(), sizeof(unsigned long long) * ntl));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));  // the host staging vectors end here
    return IRODORI_OK;
}

// Round-to-nearest-even f32 -> bf16 bits (NaN kept quiet).
static uint16_t bf16_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

int irodori_load_ctx_proj_weights(irodori_ctx* c, int layer, int text_dim, int aux_dim,
                                  const irodori_ctx_proj_weights* w) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && w && w->wk_text && w->wv_text, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(layer >= 0 && layer < g.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(text_dim > 0 && aux_dim >= 0, IRODORI_ERR_SHAPE, "text_dim must be > 0 and aux_dim >= 0");
    IRO_REQUIRE(aux_dim == 0 || (w->wk_aux && w->wv_aux), IRODORI_ERR_INVALID_ARG, "null aux projection");
    const int dims[2] = {text_dim, aux_dim};
    for (int sgm = 0; sgm < 2; sgm++)
        IRO_REQUIRE(c->ctx_dim[sgm] == 0 || c->ctx_dim[sgm] == dims[sgm], IRODORI_ERR_SHAPE,
                    "context projection input dims must match the layers already loaded");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const int HD = g.num_heads * g.head_dim;
    auto& lb = c->layers[layer];
    for (int sgm = 0; sgm < 2; sgm++) {
        const int K = dims[sgm];
        if (K == 0) continue;
        const int kpad = (K + 63) / 64 * 64;
        if (!lb.w_ctx[sgm]) IRO_TRY(dev_alloc(c, &lb.w_ctx[sgm], c->esz * (size_t)2 * HD * kpad));
        const float* src[2] = {sgm ? w->wk_aux : w->wk_text, sgm ? w->wv_aux : w->wv_text};
        std::vector<float> padded((size_t)kpad * HD, 0.f);  // Burn [d_in, kv_dim], rows past d_in zero
        for (int kv = 0; kv < 2; kv++) {
            memcpy(padded.data(), src[kv], sizeof(float) * (size_t)K * HD);
            IRO_TRY(ingest_kmajor(c, padded.data(), kpad, HD, 0,
                                  static_cast<char*>(lb.w_ctx[sgm]) + c->esz * (size_t)kv * HD * kpad));
        }
        c->ctx_dim[sgm] = K;
        c->ctx_kpad[sgm] = kpad;
    }
    lb.ctx_proj_loaded = true;
    return IRODORI_OK;
    IRO_GUARD_END
}

// build_kv_cache (attention.rs:431-501) of one batch row for every layer, on the device:
// per segment (text, then aux) one GEMM of the states against [Wk ; Wv] whose epilogue
// head-normalizes K and writes K and V^T into the row's context at the segment's key
// offset; ctx_mask = [text_mask | aux_mask].
int irodori_build_ctx_kv(irodori_ctx* c, int row, int t_text, const float* text_state, const uint8_t* text_mask,
                         int t_aux, const float* aux_state, const uint8_t* aux_mask) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c, IRODORI_ERR_INVALID_ARG, "null context");
    const auto& g = c->cfg;
    const int L = g.num_layers, H = g.num_heads, Dh = g.head_dim, HD = H * Dh;
    IRO_REQUIRE(row >= 0 && row < g.max_rows, IRODORI_ERR_INVALID_ARG, "row index out of range");
    IRO_REQUIRE(t_text >= 0 && t_aux >= 0, IRODORI_ERR_SHAPE, "segment lengths must be >= 0");
    const int t_ctx = t_text + t_aux;
    IRO_REQUIRE(t_ctx <= g.max_ctx, IRODORI_ERR_SHAPE,
                "t_ctx " + std::to_string(t_ctx) + " exceeds max_ctx " + std::to_string(g.max_ctx));
    IRO_REQUIRE(c->t_ctx < 0 || c->t_ctx == t_ctx, IRODORI_ERR_SHAPE,
                "t_ctx must match the context length already set (" + std::to_string(c->t_ctx) +
                    "); call irodori_clear_ctx_kv first");
    IRO_REQUIRE(t_text == 0 || (text_state && text_mask), IRODORI_ERR_INVALID_ARG, "null text state / mask");
    IRO_REQUIRE(t_aux == 0 || (aux_state && aux_mask), IRODORI_ERR_INVALID_ARG, "null aux state / mask");
    for (int l = 0; l < L; l++) {
        IRO_REQUIRE(c->layers[l].ctx_proj_loaded, IRODORI_ERR_NOT_LOADED,
                    "context projections of layer " + std::to_string(l) + " not loaded");
        IRO_REQUIRE(c->layers[l].loaded, IRODORI_ERR_NOT_LOADED,
                    "block weights (k_norm) of layer " + std::to_string(l) + " not loaded");
    }
    IRO_REQUIRE(t_aux == 0 || c->ctx_dim[1] > 0, IRODORI_ERR_NOT_LOADED, "no aux context projection loaded");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const int T1 = g.max_ctx > 0 ? g.max_ctx : 1, vs1 = (T1 + 63) / 64 * 64;

    // States -> compute dtype, input dim zero-padded, staged [text rows | aux rows].
    const int lens[2] = {t_text, t_aux};
    const float* states[2] = {text_state, aux_state};
    size_t off[2], total = 0;
    for (int sgm = 0; sgm < 2; sgm++) {
        off[sgm] = total;
        if (lens[sgm]) total += (size_t)lens[sgm] * c->ctx_kpad[sgm];
    }
    if (!c->ctx_state) {  // t_text + t_aux <= max_ctx rows of the wider padded input
        const int kmax = c->ctx_kpad[0] > c->ctx_kpad[1] ? c->ctx_kpad[0] : c->ctx_kpad[1];
        c->ctx_state_bytes = (size_t)T1 * kmax * c->esz;
        IRO_TRY(dev_alloc(c, &c->ctx_state, c->ctx_state_bytes));
    }
    IRO_REQUIRE(total * c->esz <= c->ctx_state_bytes, IRODORI_ERR_SHAPE, "context states exceed the staging buffer");
    std::vector<float> sf(total, 0.f);
    for (int sgm = 0; sgm < 2; sgm++)
        for (int j = 0; j < lens[sgm]; j++)
            memcpy(sf.data() + off[sgm] + (size_t)j * c->ctx_kpad[sgm], states[sgm] + (size_t)j * c->ctx_dim[sgm],
                   sizeof(float) * c->ctx_dim[sgm]);
    std::vector<uint16_t> sb;
    if (c->bf16) {
        sb.resize(total);
        for (size_t i = 0; i < total; i++) sb[i] = bf16_bits(sf[i]);
        IRO_TRY(upload(c, c->ctx_state, sb.data(), total * 2));
    } else if (total) {
        IRO_TRY(upload(c, c->ctx_state, sf.data(), total * 4));
    }
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));  // the host staging vectors end here
    std::vector<uint8_t> mask(t_ctx);
    for (int j = 0; j < t_text; j++) mask[j] = text_mask[j] ? 1 : 0;
    for (int j = 0; j < t_aux; j++) mask[t_text + j] = aux_mask[j] ? 1 : 0;

    for (int l = 0; l < L; l++) {
        auto& lb = c->layers[l];
        const size_t nk = (size_t)H * T1 * Dh, nv = (size_t)H * Dh * vs1;
        char* ck = static_cast<char*>(lb.ctx_k) + (size_t)row * nk * c->esz;
        char* cv = static_cast<char*>(lb.ctx_v) + (size_t)row * nv * c->esz;
        // Keys past t_ctx (and the V^T padding) hold zeros, as after irodori_set_ctx_kv.
        IRO_HIP_CHECK(hipMemsetAsync(ck, 0, nk * c->esz, c->stream));
        IRO_HIP_CHECK(hipMemsetAsync(cv, 0, nv * c->esz, c->stream));
        for (int sgm = 0; sgm < 2; sgm++) {
            if (lens[sgm] == 0) continue;
            int rc;
            if (c->bf16) {
                GemmArgs<bf16> ga{};
                ga.A = static_cast<const bf16*>(c->ctx_state) + off[sgm];
                ga.W = static_cast<const bf16*>(lb.w_ctx[sgm]);
                ga.M = lens[sgm]; ga.N = 2 * HD; ga.K = c->ctx_kpad[sgm]; ga.S = lens[sgm];
                ga.H = H; ga.D = g.model_dim; ga.eps = g.norm_eps; ga.k_norm = lb.k_norm;
                ga.Ck = reinterpret_cast<bf16*>(ck); ga.Cv = reinterpret_cast<bf16*>(cv);
                ga.key_off = sgm ? t_text : 0; ga.ctx_stride = T1; ga.ctx_vstride = vs1;
                rc = launch_gemm<bf16>(EPI_CTXKV, ga, c->stream);
            } else {
                GemmArgs<float> ga{};
                ga.A = static_cast<const float*>(c->ctx_state) + off[sgm];
                ga.W = static_cast<const float*>(lb.w_ctx[sgm]);
                ga.M = lens[sgm]; ga.N = 2 * HD; ga.K = c->ctx_kpad[sgm]; ga.S = lens[sgm];
                ga.H = H; ga.D = g.model_dim; ga.eps = g.norm_eps; ga.k_norm = lb.k_norm;
                ga.Ck = reinterpret_cast<float*>(ck); ga.Cv = reinterpret_cast<float*>(cv);
                ga.key_off = sgm ? t_text : 0; ga.ctx_stride = T1; ga.ctx_vstride = vs1;
                rc = launch_gemm<float>(EPI_CTXKV, ga, c->stream);
            }
            if (rc) { set_last_error("context KV gemm shape"); return IRODORI_ERR_SHAPE; }
        }
        IRO_TRY(check_launch("context KV build"));
        IRO_TRY(upload_row_mask(c, lb, row, t_ctx, mask.data()));
        lb.row_set[row] = 1;
    }
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (c->t_ctx != t_ctx) {
        c->graphs.clear();
    }
    c->t_ctx = t_ctx;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_set_ctx_kv(irodori_ctx* c, int layer, int row, int t_ctx, const float* k, const float* v,
                       const uint8_t* mask) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c, IRODORI_ERR_INVALID_ARG, "null context");
    const auto& g = c->cfg;
    IRO_REQUIRE(layer >= 0 && layer < g.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(row >= 0 && row < g.max_rows, IRODORI_ERR_INVALID_ARG, "row index out of range");
    IRO_REQUIRE(t_ctx >= 0 && t_ctx <= g.max_ctx, IRODORI_ERR_SHAPE,
                "t_ctx " + std::to_string(t_ctx) + " exceeds max_ctx " + std::to_string(g.max_ctx));
    IRO_REQUIRE(c->t_ctx < 0 || c->t_ctx == t_ctx, IRODORI_ERR_SHAPE,
                "t_ctx must match the context length already set (" + std::to_string(c->t_ctx) +
                    "); call irodori_clear_ctx_kv first");
    IRO_REQUIRE(t_ctx == 0 || (k && v && mask), IRODORI_ERR_INVALID_ARG, "null k/v/mask");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    auto& lb = c->layers[layer];
    int H = g.num_heads, Dh = g.head_dim, T = g.max_ctx > 0 ? g.max_ctx : 1;
    if (t_ctx > 0) {
        // k: [t, H, Dh] f32 -> [H, T, Dh];  v: [t, H, Dh] f32 -> V^T [H, Dh, Tp] with keys in
        // the attention kernel's A-operand order (vt_pos_bf16 / vt_pos_f32).
        int Tp = (T + 63) / 64 * 64;
        size_t nk = (size_t)H * T * Dh, nv = (size_t)H * Dh * Tp;
        auto cvt = bf16_bits;
        std::vector<float> kf(nk, 0.f), vf(nv, 0.f);
        for (int j = 0; j < t_ctx; j++) {
            int pos = vt_bf16_order(c) ? vt_pos_bf16(j) : vt_pos_f32(j);
            for (int hh = 0; hh < H; hh++)
                for (int d = 0; d < Dh; d++) {
                    size_t src = ((size_t)j * H + hh) * Dh + d;
                    kf[((size_t)hh * T + j) * Dh + d] = k[src];
                    vf[((size_t)hh * Dh + d) * Tp + pos] = v[src];
                }
        }
        std::vector<uint16_t> kb, vb;
        const void* kp = kf.data();
        const void* vp = vf.data();
        if (c->bf16) {
            kb.resize(nk);
            vb.resize(nv);
            for (size_t i = 0; i < nk; i++) kb[i] = cvt(kf[i]);
            for (size_t i = 0; i < nv; i++) vb[i] = cvt(vf[i]);
            kp = kb.data();
            vp = vb.data();
        }
        IRO_TRY(upload(c, static_cast<char*>(lb.ctx_k) + (size_t)row * nk * c->esz, kp, nk * c->esz));
        IRO_TRY(upload(c, static_cast<char*>(lb.ctx_v) + (size_t)row * nv * c->esz, vp, nv * c->esz));
        IRO_TRY(upload_row_mask(c, lb, row, t_ctx, mask));
    }
    if (c->t_ctx != t_ctx) {
        c->graphs.clear();
    }
    c->t_ctx = t_ctx;
    lb.row_set[row] = 1;
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_read_ctx_kv(irodori_ctx* c, int layer, int row, float* k, float* v, uint8_t* mask) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && k && v && mask, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(layer >= 0 && layer < g.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(row >= 0 && row < g.max_rows, IRODORI_ERR_INVALID_ARG, "row index out of range");
    IRO_REQUIRE(c->t_ctx >= 0 && c->layers[layer].row_set[row], IRODORI_ERR_NOT_LOADED,
                "context KV of this layer / row not set");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    auto& lb = c->layers[layer];
    const int H = g.num_heads, Dh = g.head_dim, T = g.max_ctx > 0 ? g.max_ctx : 1, Tp = (T + 63) / 64 * 64;
    const size_t nk = (size_t)H * T * Dh, nv = (size_t)H * Dh * Tp;
    std::vector<unsigned char> kb(nk * c->esz), vb(nv * c->esz);
    std::vector<float> mf(T);
    IRO_HIP_CHECK(hipMemcpyAsync(kb.data(), static_cast<char*>(lb.ctx_k) + (size_t)row * nk * c->esz, kb.size(),
                                 hipMemcpyDeviceToHost, c->stream));
    IRO_HIP_CHECK(hipMemcpyAsync(vb.data(), static_cast<char*>(lb.ctx_v) + (size_t)row * nv * c->esz, vb.size(),
                                 hipMemcpyDeviceToHost, c->stream));
    IRO_HIP_CHECK(hipMemcpyAsync(mf.data(), lb.ctx_mask + (size_t)row * T, sizeof(float) * T,
                                 hipMemcpyDeviceToHost, c->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    auto at = [&](const std::vector<unsigned char>& b, size_t i) -> float {
        if (!c->bf16) {
            float f;
            memcpy(&f, b.data() + 4 * i, 4);
            return f;
        }
        uint32_t u = (uint32_t)(b[2 * i] | (b[2 * i + 1] << 8)) << 16;
        float f;
        memcpy(&f, &u, 4);
        return f;
    };
    for (int j = 0; j < c->t_ctx; j++) {
        const int pos = vt_bf16_order(c) ? vt_pos_bf16(j) : vt_pos_f32(j);
        for (int hh = 0; hh < H; hh++)
            for (int d = 0; d < Dh; d++) {
                const size_t dst = ((size_t)j * H + hh) * Dh + d;
                k[dst] = at(kb, ((size_t)hh * T + j) * Dh + d);
                v[dst] = at(vb, ((size_t)hh * Dh + d) * Tp + pos);
            }
        mask[j] = mf[j] != 0.f;
    }
    return IRODORI_OK;
    IRO_GUARD_END
}

// Upload a latent key mask [B, S] (nonzero = the key attends) as per-row tile validity
// words and a float mask, and route it to the attention launches until the guard ends.
static int upload_latent_mask(irodori_ctx* c, int B, int S, const uint8_t* mask) {
    const int ntl = (S + 63) / 64;
    std::vector<unsigned long long> bits((size_t)B * ntl, 0ull);
    std::vector<float> mf((size_t)B * S, 0.f);
    for (int b = 0; b < B; b++)
        for (int s = 0; s < S; s++)
            if (mask[(size_t)b * S + s]) {
                bits[(size_t)b * ntl + s / 64] |= 1ull << (s % 64);
                mf[(size_t)b * S + s] = 1.f;
            }
    IRO_TRY(upload(c, c->lat_bits, bits.data(), sizeof(unsigned long long) * bits.size()));
    IRO_TRY(upload(c, c->lat_mask_f, mf.data(), sizeof(float) * mf.size()));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));  // the host staging vectors end here
    return IRODORI_OK;
}

struct LatentMaskScope {
    irodori_ctx* c;
    LatentMaskScope(irodori_ctx* ctx, bool on) : c(ctx) { c->lat_on = on; }
    ~LatentMaskScope() { c->lat_on = false; }
};

static int forward_impl(irodori_ctx* c, int B, int S, const float* x_t, const float* t, const uint8_t* latent_mask,
                 float* v_out, float* debug);

int irodori_forward(irodori_ctx* c, int B, int S, const float* x_t, const float* t, float* v_out, float* debug) {
    return forward_impl(c, B, S, x_t, t, nullptr, v_out, debug);
}

int irodori_forward_masked(irodori_ctx* c, int B, int S, const float* x_t, const float* t, const uint8_t* latent_mask,
                           float* v_out, float* debug) {
    return forward_impl(c, B, S, x_t, t, latent_mask, v_out, debug);
}

static int forward_impl(irodori_ctx* c, int B, int S, const float* x_t, const float* t, const uint8_t* latent_mask,
                 float* v_out, float* debug) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && x_t && t && v_out, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(B > 0 && B <= g.max_rows, IRODORI_ERR_SHAPE, "batch out of range [1, max_rows]");
    IRO_REQUIRE(S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE, "seq out of range [1, max_seq]");
    IRO_TRY(check_ready(c, B));
    IRO_HIP_CHECK(hipSetDevice(c->device));
    int D = g.model_dim, P = g.latent_dim, L = g.num_layers;
    if (latent_mask) IRO_TRY(upload_latent_mask(c, B, S, latent_mask));
    LatentMaskScope lms(c, latent_mask != nullptr);
    IRO_TRY(ensure_nvec(c, B));
    IRO_TRY(upload(c, c->tvec, t, sizeof(float) * B));
    IRO_TRY(upload(c, c->xt, x_t, sizeof(float) * (size_t)B * S * P));
    RoctxRange fwd("dit_forward_with_cond_fused");
    IRO_TRY(enqueue_mod_table(c, B, false));
    ModTable mt{c->tab, c->zero_step, 0, 1, L};
    {
        RoctxRange range("in_proj");
        IRO_TRY(enqueue_inproj(c, B, S, c->xt, B, 0, mt, c->stream));
    }
    size_t n = (size_t)B * S * D;
    if (debug) IRO_HIP_CHECK(hipMemcpyAsync(debug, c->x, sizeof(float) * n, hipMemcpyDeviceToHost, c->stream));
    for (int l = 0; l < L; l++) {
        IRO_TRY(enqueue_layer_any(c, l, B, S, mt));
        if (debug)
            IRO_HIP_CHECK(hipMemcpyAsync(debug + (size_t)(l + 1) * n, c->x, sizeof(float) * n, hipMemcpyDeviceToHost,
                                         c->stream));
    }
    {
        RoctxRange range("out_proj");  // out_norm folded into the head's weights (dit/model.rs:391-392)
        IRO_TRY(enqueue_head(c, B, S, 0, c->stream));
    }
    IRO_HIP_CHECK(hipMemcpyAsync(v_out, c->vout, sizeof(float) * (size_t)B * S * P, hipMemcpyDeviceToHost, c->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    return IRODORI_OK;
    IRO_GUARD_END
}

int irodori_block_forward(irodori_ctx* c, int layer, int B, int S, float* x, const float* cond) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && x && cond, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(layer >= 0 && layer < g.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(B > 0 && B <= g.max_rows && S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE, "batch/seq out of range");
    IRO_REQUIRE(c->layers[layer].loaded, IRODORI_ERR_NOT_LOADED, "block weights not loaded");
    if (c->t_ctx > 0)
        for (int r = 0; r < B; r++)
            IRO_REQUIRE(c->layers[layer].row_set[r], IRODORI_ERR_NOT_LOADED, "context KV not set for a row");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    int D = g.model_dim, L = g.num_layers;
    IRO_TRY(ensure_nvec(c, B));
    IRO_TRY(upload(c, c->cond, cond, sizeof(float) * (size_t)B * 3 * D));
    IRO_TRY(enqueue_mod_table(c, B, true, layer, layer + 1));
    ModTable mt{c->tab, c->zero_step, 0, 1, L};
    size_t n = (size_t)B * S * D;
    IRO_TRY(upload(c, c->x, x, sizeof(float) * n));
    if (fused_for(c, mt, B)) {
        launch_mod_stats<bf16>(c->x, static_cast<bf16*>(c->h), B * S, S, D, mt, layer, 0, c->rstat, c->stream);
    } else if (c->bf16) {
        launch_norm_mod<bf16>(c->x, c->fp8 ? nullptr : static_cast<bf16*>(c->h), B * S, S, D, g.norm_eps, mt, layer,
                              0, c->stream, c->fp8 ? c->h8 : nullptr, c->fp8 ? c->h8s : nullptr);
    } else
        launch_norm_mod<float>(c->x, static_cast<float*>(c->h), B * S, S, D, g.norm_eps, mt, layer, 0, c->stream);
    IRO_TRY(enqueue_layer_any(c, layer, B, S, mt));
    IRO_HIP_CHECK(hipMemcpyAsync(x, c->x, sizeof(float) * n, hipMemcpyDeviceToHost, c->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    return IRODORI_OK;
    IRO_GUARD_END
}

static int sample_device_impl(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const int32_t* lengths,
                       const float* d_x0, float* d_x_out);

int irodori_sample_device(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const float* d_x0,
                          float* d_x_out) {
    return sample_device_impl(c, p, U, S, nullptr, d_x0, d_x_out);
}

int irodori_sample_device_masked(irodori_ctx* c, const irodori_sampler_params* p, int U, int S,
                                 const int32_t* lengths, const float* d_x0, float* d_x_out) {
    if (!lengths) {
        set_last_error("null lengths");
        return IRODORI_ERR_INVALID_ARG;
    }
    return sample_device_impl(c, p, U, S, lengths, d_x0, d_x_out);
}

// Restores the context's speaker-KV routing when a sampling call ends.
struct KvsScope {
    irodori_ctx* c;
    ~KvsScope() { c->kvs_on = false; }
};

// lengths (nullable, host [U]): utterance u attends to its first lengths[u] latent keys
// in every role (padded variable-length batches).
static int sample_device_impl(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const int32_t* lengths,
                       const float* d_x0, float* d_x_out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && p && d_x0 && d_x_out, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_TRY(validate_params(p));
    const auto& g = c->cfg;
    float scales[3];
    const int n = cfg_signals(p, scales);
    const int R = cfg_roles(p, n);
    const int B = R * U;
    IRO_REQUIRE(U > 0 && B <= g.max_rows, IRODORI_ERR_SHAPE,
                std::to_string(R) + " roles x " + std::to_string(U) + " utterances exceed max_rows");
    IRO_REQUIRE(S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE, "seq out of range [1, max_seq]");
    IRO_TRY(check_ready(c, B));
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const int N = p->num_steps, P = g.latent_dim, L = g.num_layers;
    const int method = p->method, mode = p->cfg_mode;
    const bool heun = method == IRODORI_METHOD_HEUN, plms = method == IRODORI_METHOD_PLMS4;
    if (lengths) {
        std::vector<uint8_t> m((size_t)B * S, 0);
        for (int u = 0; u < U; u++) {
            IRO_REQUIRE(lengths[u] >= 1 && lengths[u] <= S, IRODORI_ERR_SHAPE, "utterance length must be in [1, seq]");
            for (int r = 0; r < R; r++)
                for (int s2 = 0; s2 < lengths[u]; s2++) m[(size_t)(r * U + u) * S + s2] = 1;
        }
        IRO_TRY(upload_latent_mask(c, B, S, m.data()));
    }
    LatentMaskScope lms(c, lengths != nullptr);

    // Schedule t_i = 0.999 (1 - i/N) in f32 (euler_sampler.rs:325-328), the CFG window
    // (:379), and one planned evaluation per step (two for Heun, the corrector at t_{i+1}).
    std::vector<float> ts(N + 1);
    for (int i = 0; i <= N; i++) ts[i] = 0.999f * (1.0f - (float)i / (float)N);
    auto cfg_at = [&](float t) { return n > 0 && p->min_t <= t && t <= p->max_t; };
    std::vector<RfEval> plan((size_t)2 * N);
    std::vector<int> roles_of((size_t)2 * N, 0);
    auto fill = [&](int e, float t, float dt, bool on, int step) {
        RfEval& ev = plan[e];
        ev = RfEval{};
        ev.dt = dt;
        int roles = 1;
        if (on) {
            if (mode == IRODORI_CFG_JOINT) {
                ev.nterm = 1; ev.role[0] = 1; ev.scale[0] = scales[0];
            } else if (mode == IRODORI_CFG_INDEPENDENT) {
                ev.nterm = n;
                for (int k = 0; k < n; k++) { ev.role[k] = 1 + k; ev.scale[k] = scales[k]; }
            } else {  // Alternating: the dropped signal cycles with the step (:472-473)
                const int a = step % n;
                ev.nterm = 1; ev.role[0] = 1 + a; ev.scale[0] = scales[a];
            }
            for (int k = 0; k < ev.nterm; k++) roles |= 1 << ev.role[k];
        }
        if (p->has_temporal_rescale && t < 1.0f) {
            // math.rs:38-53, scalars in f32
            const float omt = 1.0f - t;
            const float snr = (omt * omt) / (t * t);
            const float sig2 = p->rescale_sigma * p->rescale_sigma;
            ev.rescale = 1;
            ev.omt = omt;
            ev.ratio = (snr * sig2 + 1.0f) / (snr * sig2 / p->rescale_k + 1.0f);
        }
        roles_of[e] = roles;
    };
    bool spk_active = p->has_speaker_kv != 0;  // speaker_kv.is_some() (:337)
    int revert_step = -1, nhist = 0;
    int prev_cfg = cfg_at(ts[0]), prev_spk = spk_active;
    for (int i = 0; i < N; i++) {
        const float t = ts[i], tn = ts[i + 1];
        const bool on = cfg_at(t);
        if (plms && (on != (bool)prev_cfg || spk_active != (bool)prev_spk)) {  // (:383-390)
            nhist = 0;
            prev_cfg = on;
            prev_spk = spk_active;
        }
        fill(2 * i, t, tn - t, on, i);
        if (spk_active && p->has_speaker && p->speaker_kv_has_min_t && tn < p->speaker_kv_min_t &&
            t >= p->speaker_kv_min_t) {  // (:533-545), before the corrector
            revert_step = i;
            spk_active = false;
        }
        if (plms) {
            nhist = nhist < 4 ? nhist + 1 : 4;
            plan[2 * i].ab_order = nhist;
        }
        if (heun) fill(2 * i + 1, tn, tn - t, cfg_at(tn), i);
    }

    // Modulation vectors for every t_i (i <= N: the corrector's t_{i+1}), the plan.
    IRO_TRY(ensure_nvec(c, N + 1));
    if (N > c->plan_cap) {
        IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
        IRO_TRY(dalloc(c, &c->plan, sizeof(RfEval) * 2 * (size_t)N));
        c->plan_cap = N;
        c->graphs.clear();
    }
    IRO_TRY(upload(c, c->plan, plan.data(), sizeof(RfEval) * plan.size()));
    IRO_TRY(upload(c, c->tvec, ts.data(), sizeof(float) * (N + 1)));
    IRO_TRY(enqueue_mod_table(c, N + 1, false));

    // Speaker-KV scaling (euler_sampler.rs:258-264, :294-300): the conditioned rows, or in
    // Independent mode every row of the batched cache, in the first max_layers layers.
    const bool kvs = p->has_speaker_kv && p->has_speaker && c->t_ctx > 0;
    const int nl = p->speaker_kv_max_layers < 0 || p->speaker_kv_max_layers > L ? L : p->speaker_kv_max_layers;
    const int rows_scaled = mode == IRODORI_CFG_INDEPENDENT ? B : U;
    const int T1 = g.max_ctx > 0 ? g.max_ctx : 1, vs1 = (T1 + 63) / 64 * 64;
    KvsScope kscope{c};
    auto scale_kv = [&](bool from_ctx, float factor) -> int {
        for (int l = 0; l < nl; l++) {
            auto& lb = c->layers[l];
            const void* sk = from_ctx ? lb.ctx_k : c->act_k[l];
            const void* sv = from_ctx ? lb.ctx_v : c->act_v[l];
            if (c->bf16)
                launch_scale_ctx_aux<bf16>(static_cast<const bf16*>(sk), static_cast<const bf16*>(sv),
                                           static_cast<bf16*>(c->act_k[l]), static_cast<bf16*>(c->act_v[l]), B,
                                           rows_scaled, g.num_heads, g.head_dim, vt_bf16_order(c), T1, vs1,
                                           c->t_ctx, p->ctx_aux_start, factor, c->stream);
            else
                launch_scale_ctx_aux<float>(static_cast<const float*>(sk), static_cast<const float*>(sv),
                                            static_cast<float*>(c->act_k[l]), static_cast<float*>(c->act_v[l]), B,
                                            rows_scaled, g.num_heads, g.head_dim, false, T1, vs1, c->t_ctx,
                                            p->ctx_aux_start, factor, c->stream);
        }
        return check_launch("speaker kv scaling");
    };
    if (kvs) {
        IRO_REQUIRE(p->ctx_aux_start >= 0 && p->ctx_aux_start <= c->t_ctx, IRODORI_ERR_CONFIG,
                    "ctx_aux_start must be in [0, t_ctx]");
        if ((int)c->act_k.size() < L) {
            IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
            const size_t kb = (size_t)g.max_rows * g.num_heads * T1 * g.head_dim * c->esz;
            const size_t vb = (size_t)g.max_rows * g.num_heads * g.head_dim * vs1 * c->esz;
            c->act_k.assign(L, nullptr);
            c->act_v.assign(L, nullptr);
            // Zeroed once: the V^T padding columns past max_ctx (which the scaling never
            // writes) must hold finite values, like the context buffers they mirror.
            for (int l = 0; l < L; l++) {
                IRO_TRY(dev_alloc(c, &c->act_k[l], kb));
                IRO_TRY(dev_alloc(c, &c->act_v[l], vb));
                IRO_HIP_CHECK(hipMemsetAsync(c->act_k[l], 0, kb, c->stream));
                IRO_HIP_CHECK(hipMemsetAsync(c->act_v[l], 0, vb, c->stream));
            }
        }
        IRO_TRY(scale_kv(true, p->speaker_kv_scale));
        c->kvs_on = true;
        c->kvs_layers = nl;
    }

    launch_scale_copy(d_x0, c->xt, U * S * P, p->has_truncation ? p->truncation_factor : 1.0f, c->stream);
    IRO_HIP_CHECK(hipMemsetAsync(c->step, 0, 2 * sizeof(int), c->stream));
    IRO_TRY(check_launch("sampler setup"));

    // One captured graph per distinct evaluation (roles, phase), replayed per step.
    auto graph_for = [&](int roles, int phase, hipGraphExec_t* out) -> int {
        GraphKey key{U, S, c->t_ctx, roles, method, phase, lengths ? 1 : 0, c->kvs_on ? c->kvs_layers : 0};
        if (hipGraphExec_t hit = c->graphs.find(key)) {
            *out = hit;
            return IRODORI_OK;
        }
        hipGraph_t graph = nullptr;
        IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
        IRO_HIP_CHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_eval(c, U, S, roles, method, phase, phase == 1 ? c->xin : c->xt);
        hipError_t ee = hipStreamEndCapture(c->stream, &graph);
        if (rc != IRODORI_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (ee != hipSuccess) {
            set_last_error(std::string("graph capture: ") + hipGetErrorString(ee));
            return IRODORI_ERR_HIP;
        }
        hipGraphExec_t exec = nullptr;
        ee = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (ee != hipSuccess) {
            set_last_error(std::string("graph instantiate: ") + hipGetErrorString(ee));
            return IRODORI_ERR_HIP;
        }
        c->graphs.insert(key, exec);
        *out = exec;
        return IRODORI_OK;
    };
    // One range per evaluation, named as the reference's (euler_sampler.rs:409-515, :580):
    // several roles batched, the conditioned role alone, or one dropped-signal role alone.
    auto eval_name = [](int roles) {
        return (roles & (roles - 1)) ? "forward_batched_cfg" : roles == 1 ? "forward_cond" : "forward_uncond";
    };
    for (int i = 0; i < N; i++) {
        hipGraphExec_t ex = nullptr;
        {
            RoctxRange range(eval_name(roles_of[2 * i]));
            IRO_TRY(graph_for(roles_of[2 * i], 0, &ex));
            IRO_HIP_CHECK(hipGraphLaunch(ex, c->stream));
        }
        if (i == revert_step && kvs) IRO_TRY(scale_kv(false, 1.0f / p->speaker_kv_scale));
        if (heun) {
            RoctxRange range("heun_corrector");
            IRO_TRY(graph_for(roles_of[2 * i + 1], 1, &ex));
            IRO_HIP_CHECK(hipGraphLaunch(ex, c->stream));
        }
    }
    IRO_HIP_CHECK(hipMemcpyAsync(d_x_out, c->xt, sizeof(float) * (size_t)U * S * P, hipMemcpyDeviceToDevice, c->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    return IRODORI_OK;
    IRO_GUARD_END
}

static int sample_host(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const int32_t* lengths,
                const float* x0, float* x_out);

int irodori_sample(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const float* x0, float* x_out) {
    return sample_host(c, p, U, S, nullptr, x0, x_out);
}

int irodori_sample_masked(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const int32_t* lengths,
                          const float* x0, float* x_out) {
    if (!lengths) {
        set_last_error("null lengths");
        return IRODORI_ERR_INVALID_ARG;
    }
    return sample_host(c, p, U, S, lengths, x0, x_out);
}

static int sample_host(irodori_ctx* c, const irodori_sampler_params* p, int U, int S, const int32_t* lengths,
                const float* x0, float* x_out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && p && x0 && x_out, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_TRY(validate_params(p));
    const auto& g = c->cfg;
    IRO_REQUIRE(U > 0 && U <= g.max_rows && S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE, "utterances/seq out of range");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    size_t n = (size_t)U * S * g.latent_dim;
    // Staged through the Heun predictor buffer: the sampler reads x0 before its first
    // evaluation and writes x_out after its last.
    IRO_TRY(upload(c, c->xin, x0, sizeof(float) * n));
    int rc = sample_device_impl(c, p, U, S, lengths, c->xin, c->xin);
    if (rc != IRODORI_OK) return rc;
    IRO_HIP_CHECK(hipMemcpy(x_out, c->xin, sizeof(float) * n, hipMemcpyDeviceToHost));
    return IRODORI_OK;
    IRO_GUARD_END
}

// ---- isolated block operators (the model's kernels on a loaded context) -----------------

int irodori_op_joint_attention(irodori_ctx* c, int layer, int B, int S, const float* q, const float* k,
                               const float* v, const float* gate, float* out, void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && q && k && v && out, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(layer >= 0 && layer < g.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(B > 0 && B <= g.max_rows && S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE,
                "batch must be in [1, max_rows], seq in [1, max_seq]");
    IRO_REQUIRE(!c->fp8, IRODORI_ERR_DTYPE, "the joint attention operator runs bf16 or f32 contexts");
    IRO_REQUIRE(g.head_dim == 64, IRODORI_ERR_SHAPE, "the joint attention operator takes 64-dim heads");
    IRO_REQUIRE(c->layers[layer].loaded, IRODORI_ERR_NOT_LOADED, "block weights of the layer not loaded");
    if (c->t_ctx > 0)
        for (int r = 0; r < B; r++)
            IRO_REQUIRE(c->layers[layer].row_set[r], IRODORI_ERR_NOT_LOADED,
                        "context KV of row " + std::to_string(r) + " not set");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
    const int H = g.num_heads, D = g.model_dim, vt = (S + 63) / 64 * 64;
    const float q_scale = 1.4426950408889634f / sqrtf((float)g.head_dim);
    auto& lb = c->layers[layer];
    ModTable mt{c->tab, c->zero_step, 0, B, g.num_layers};  // not read by the attention
    if (c->bf16) {
        launch_attn_op_stage<bf16>(q, k, v, gate, lb.q_norm, lb.k_norm, c->rope_cos, c->rope_sin, B, S, H, g.norm_eps,
                                   q_scale, vt, static_cast<bf16*>(c->q), static_cast<bf16*>(c->ks),
                                   static_cast<bf16*>(c->vs), static_cast<bf16*>(c->gate), st);
        IRO_TRY(enqueue_part<bf16>(c, layer, B, S, mt, PART_ATTN, 0, st));
        launch_to_f32<bf16>(static_cast<const bf16*>(c->o), (long)B * S * D, out, st);
    } else {
        launch_attn_op_stage<float>(q, k, v, gate, lb.q_norm, lb.k_norm, c->rope_cos, c->rope_sin, B, S, H,
                                    g.norm_eps, q_scale, vt, static_cast<float*>(c->q), static_cast<float*>(c->ks),
                                    static_cast<float*>(c->vs), static_cast<float*>(c->gate), st);
        IRO_TRY(enqueue_part<float>(c, layer, B, S, mt, PART_ATTN, 0, st));
        launch_to_f32<float>(static_cast<const float*>(c->o), (long)B * S * D, out, st);
    }
    return check_launch("joint attention operator");
    IRO_GUARD_END
}

int irodori_op_swiglu_mlp(irodori_ctx* c, int layer, int B, int S, float* x, const float* shift, const float* scale,
                          const float* gate, void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && x && shift && scale && gate, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(layer >= 0 && layer < g.num_layers, IRODORI_ERR_INVALID_ARG, "layer index out of range");
    IRO_REQUIRE(B > 0 && B <= g.max_rows && S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE,
                "batch must be in [1, max_rows], seq in [1, max_seq]");
    IRO_REQUIRE(c->layers[layer].loaded, IRODORI_ERR_NOT_LOADED, "block weights of the layer not loaded");
    IRO_HIP_CHECK(hipSetDevice(c->device));
    const int D = g.model_dim, L = g.num_layers;
    IRO_TRY(ensure_nvec(c, B));
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : c->stream;
    // The caller's vectors in table rows 0..B-1 of (layer, mlp); the table is rebuilt by
    // the next forward or sampling call.
    launch_put_mod_vectors(shift, scale, gate, B, D, L, layer, 1, c->tab, st);
    PartOpts opt;
    opt.no_next = true;
    const ModTable one{c->tab, c->zero_step, 0, 1, L};
    if (c->bf16 && fused_for(c, one, 1)) {
        // The sampler chain's form, one batch row per launch (each on its own vector): the
        // operand x (1 + scale) and the row sums, then W1|W3 with the norm folded in and W2
        // with the gated residual.
        const int cap = c->nvec_cap, F = c->Fp;
        bf16* stage = static_cast<bf16*>(c->shift_stage);
        launch_shift_stage(c->tab, B, cap, L, D, stage, st);
        GemmArgs<bf16> ga{};
        ga.A = stage + (size_t)(layer * 2 + 1) * cap * D;
        ga.W = static_cast<const bf16*>(c->layers[layer].w13);
        ga.w_tiled = c->w_tiled;
        ga.M = B;
        ga.N = 2 * F;
        ga.K = D;
        ga.S = B;
        ga.C = c->bias13 + (size_t)layer * cap * 2 * F;
        IRO_REQUIRE(launch_gemm<bf16>(EPI_STORE, ga, st) == 0, IRODORI_ERR_SHAPE, "shift bias gemm shape");
        for (int b = 0; b < B; b++) {
            ModTable mt{c->tab, c->zero_step, 0, 1, L, 0, b};
            const size_t tok0 = (size_t)b * S;
            opt.x = x + tok0 * D;
            launch_mod_stats<bf16>(opt.x, static_cast<bf16*>(c->h) + tok0 * D, S, S, D, mt, layer, 1,
                                   c->rstat + tok0 * (D / 32), st);
            IRO_TRY(enqueue_part<bf16>(c, layer, 1, S, mt, PART_W13, b, st, opt));
            IRO_TRY(enqueue_part<bf16>(c, layer, 1, S, mt, PART_W2, b, st, opt));
        }
    } else {
        // All rows in one launch set, each row on its own vector (rows_per_vec 1): the adaLN
        // kernel, W1|W3 with the SwiGLU epilogue, W2 with the gated residual.
        opt.x = x;
        for (int part : {PART_NORM_MLP, PART_W13, PART_W2}) {
            if (c->bf16)
                IRO_TRY(enqueue_part<bf16>(c, layer, B, S, one, part, 0, st, opt));
            else
                IRO_TRY(enqueue_part<float>(c, layer, B, S, one, part, 0, st, opt));
        }
    }
    return check_launch("swiglu mlp operator");
    IRO_GUARD_END
}

int irodori_profile_layer(irodori_ctx* c, int B, int S, int iters, irodori_kernel_times* out) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(c && out, IRODORI_ERR_INVALID_ARG, "null argument");
    const auto& g = c->cfg;
    IRO_REQUIRE(B > 0 && B <= g.max_rows && S > 0 && S <= g.max_seq, IRODORI_ERR_SHAPE,
                "batch must be in [1, max_rows], seq in [1, max_seq]");
    IRO_REQUIRE(iters > 0, IRODORI_ERR_INVALID_ARG, "iters must be > 0");
    IRO_REQUIRE(c->bf16, IRODORI_ERR_DTYPE, "irodori_profile_layer times the bf16 / fp8 path");
    IRO_TRY(check_ready(c, B));
    IRO_HIP_CHECK(hipSetDevice(c->device));
    int L = g.num_layers;
    // One modulation vector (t = 0.5) shared by every row, as in a sampler evaluation; the
    // state from one in_proj of ones and one pass over the blocks.
    std::vector<float> t(1, 0.5f), x0((size_t)B * S * g.latent_dim, 1.0f);
    IRO_TRY(ensure_nvec(c, 1));
    IRO_TRY(upload(c, c->tvec, t.data(), sizeof(float)));
    IRO_TRY(upload(c, c->xt, x0.data(), sizeof(float) * x0.size()));
    IRO_TRY(enqueue_mod_table(c, 1, false));
    ModTable mt{c->tab, c->zero_step, 0, B, L};
    IRO_TRY(enqueue_inproj(c, B, S, c->xt, B, 0, mt, c->stream));
    for (int l = 0; l < L; l++) IRO_TRY(enqueue_layer_any(c, l, B, S, mt));  // fills every operand
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));

    // The adaLN kernel is HBM-bound: time it on a pool of distinct (x, h) buffer pairs larger
    // than the L2 and the MALL together (>= 640 MB), one pair per launch, so that every launch
    // reads x from and writes h to HBM rather than to a warm cache.
    const size_t xb = (size_t)B * S * g.model_dim * sizeof(float), hb = (size_t)B * S * g.model_dim * sizeof(bf16);
    const size_t kPoolBytes = (size_t)640 << 20;
    const int npair = (int)std::max<size_t>(1, (kPoolBytes + xb + hb - 1) / (xb + hb));
    struct PoolGuard {
        char* p = nullptr;
        hipStream_t st;
        ~PoolGuard() {
            if (p) {
                (void)hipStreamSynchronize(st);
                (void)hipFree(p);
            }
        }
    } pg{nullptr, c->stream};
    IRO_HIP_CHECK(hipMalloc(&pg.p, (xb + hb) * (size_t)npair));
    char* const pool = pg.p;
    IRO_HIP_CHECK(hipMemsetAsync(pool, 0x3c, (xb + hb) * (size_t)npair, c->stream));
    IRO_HIP_CHECK(hipStreamSynchronize(c->stream));
    hipEvent_t e0, e1;
    IRO_HIP_CHECK(hipEventCreate(&e0));
    IRO_HIP_CHECK(hipEventCreate(&e1));
    float* outs[7] = {&out->norm_mod_us, &out->qkvg_gemm_us, &out->attention_us, &out->wo_gemm_us,
                      &out->w13_gemm_us, &out->w2_gemm_us, &out->final_us};
    static const int part_of[6] = {-1, PART_QKVG, PART_ATTN, PART_WO, PART_W13, PART_W2};
    int rc = IRODORI_OK;
    for (int kidx = 0; kidx < 7 && rc == IRODORI_OK; kidx++) {
        (void)hipEventRecord(e0, c->stream);
        for (int it = 0; it < iters && rc == IRODORI_OK; it++) {
            // Launch `it` uses layer it % L: the weights (and context K / V) cycle through all
            // layers, as the blocks of an RF step read them.
            const int l = it % L;
            if (kidx == 6) {
                rc = enqueue_head(c, B, S, 0, c->stream);
            } else if (kidx == 0) {
                // The unfused adaLN kernel (forwards whose rows carry different t, f32, fp8).
                char* pair = pool + (xb + hb) * (size_t)(it % npair);
                launch_norm_mod<bf16>(reinterpret_cast<const float*>(pair), reinterpret_cast<bf16*>(pair + xb),
                                      B * S, S, g.model_dim, g.norm_eps, mt, l, 1, c->stream);
            } else {
                rc = enqueue_part<bf16>(c, l, B, S, mt, part_of[kidx], 0, c->stream);
            }
        }
        (void)hipEventRecord(e1, c->stream);
        hipError_t se = hipEventSynchronize(e1);
        float ms = 0.f;
        if (se == hipSuccess) se = hipEventElapsedTime(&ms, e0, e1);
        if (se != hipSuccess && rc == IRODORI_OK) {
            set_last_error(std::string("profile events: ") + hipGetErrorString(se));
            rc = IRODORI_ERR_HIP;
        }
        *outs[kidx] = ms * 1000.f / (float)iters;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != IRODORI_OK) return rc;
    // The operands the timed launches overwrote are restored by the next forward (in_proj
    // rewrites the state); nothing else depends on them.
    return check_launch("profile");
    IRO_GUARD_END
}

// ---- operator entry points ------------------------------------------------------------

int irodori_op_mx_quantize(const float* x, int rows, int dim, uint8_t* q, uint8_t* s, void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(x && q && s, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(rows > 0 && dim > 0 && dim % 32 == 0, IRODORI_ERR_SHAPE, "mx_quantize requires rows > 0 and dim % 32 == 0");
    launch_mx_quant_rows<float>(x, rows, dim, q, s, static_cast<hipStream_t>(stream));
    return check_launch("mx_quantize");
    IRO_GUARD_END
}

int irodori_op_gemm_fp8(const uint8_t* a8, const uint8_t* a_scale, const uint8_t* w8, const float* w_scale, int M,
                        int N, int K, float* c, void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(a8 && a_scale && w8 && w_scale && c, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(M > 0 && N > 0 && N % 64 == 0 && K > 0 && K % 128 == 0 && K <= 8192, IRODORI_ERR_SHAPE,
                "gemm_fp8 requires M > 0, N % 64 == 0 and K % 128 == 0 (K <= 8192)");
    GemmArgs<bf16> ga{};
    ga.A8 = a8;
    ga.As = a_scale;
    ga.W8 = w8;
    ga.ws = w_scale;
    ga.M = M;
    ga.N = N;
    ga.K = K;
    ga.C = c;
    if (launch_gemm_fp8(EPI_STORE, ga, static_cast<hipStream_t>(stream))) {
        set_last_error("gemm_fp8 launch rejected the shape");
        return IRODORI_ERR_SHAPE;
    }
    return check_launch("gemm_fp8");
    IRO_GUARD_END
}

int irodori_op_rms_norm(const float* x, const float* w, int rows, int dim, float eps, float* y, void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(x && w && y, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(rows > 0 && dim > 0, IRODORI_ERR_SHAPE, "RMSNorm requires rows > 0 and dim > 0");
    launch_rms_norm_op(x, w, rows, dim, eps, y, static_cast<hipStream_t>(stream));
    return check_launch("rms_norm");
    IRO_GUARD_END
}

int irodori_op_fused_adaln(const float* x, const float* scale, const float* shift, int batch, int seq, int dim,
                           float eps, float* y, void* stream) {
    IRO_GUARD_BEGIN
    IRO_REQUIRE(x && scale && shift && y, IRODORI_ERR_INVALID_ARG, "null argument");
    IRO_REQUIRE(batch > 0 && seq > 0 && dim > 0, IRODORI_ERR_SHAPE, "fused AdaLN requires positive dims");
    launch_fused_adaln_op(x, scale, shift, batch, seq, dim, eps, y, static_cast<hipStream_t>(stream));
    return check_launch("fused_adaln");
    IRO_GUARD_END
}

}  // extern "C"
