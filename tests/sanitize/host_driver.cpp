// Host-code sanitizer driver: calls the C ABI's device-free host logic (argument and
// config validation, the sampler-parameter rules, the error plumbing, the roctx switch)
// of a library whose host code is built with AddressSanitizer and UBSan
// (tests/sanitize/Makefile).  Exits 0 when every call returns the expected status; a
// sanitizer report aborts the process.  No GPU is needed: every call fails or returns
// before its first device call, as on a host without one.
#include <cmath>
#include <cstdio>
#include <cstring>

#include "irodori_hip.h"

static int failures = 0;

static void expect(const char* what, int got, int want) {
    const char* msg = irodori_last_error();
    if (got != want) {
        std::printf("FAIL %s: got %d want %d (%s)\n", what, got, want, msg ? msg : "");
        failures++;
    }
}

static irodori_sampler_params joint(int steps) {
    irodori_sampler_params p{};
    p.num_steps = steps;
    p.method = IRODORI_METHOD_EULER;
    p.cfg_mode = IRODORI_CFG_JOINT;
    p.scale_text = 3.f;
    p.scale_speaker = 3.f;
    p.min_t = 0.f;
    p.max_t = 1.f;
    p.has_speaker = 1;
    p.truncation_factor = 1.f;
    p.rescale_k = 1.f;
    p.rescale_sigma = 1.f;
    p.speaker_kv_scale = 1.f;
    p.speaker_kv_max_layers = -1;
    return p;
}

int main() {
    if (!irodori_version() || !std::strlen(irodori_version())) failures++;
    expect("roctx off by default", irodori_roctx_enabled(), 0);

    irodori_sampler_params p = joint(40);
    expect("valid joint params", irodori_sampler_params_validate(&p), IRODORI_OK);
    expect("null params", irodori_sampler_params_validate(nullptr), IRODORI_ERR_INVALID_ARG);
    p = joint(0);
    expect("zero steps", irodori_sampler_params_validate(&p), IRODORI_ERR_CONFIG);
    p = joint(10);
    p.scale_speaker = 2.f;
    expect("joint unequal scales", irodori_sampler_params_validate(&p), IRODORI_ERR_CONFIG);
    p = joint(10);
    p.min_t = NAN;
    expect("nan min_t", irodori_sampler_params_validate(&p), IRODORI_ERR_CONFIG);
    p = joint(10);
    p.method = 9;
    expect("unknown method", irodori_sampler_params_validate(&p), IRODORI_ERR_CONFIG);

    irodori_ctx* ctx = nullptr;
    expect("null config", irodori_ctx_create(0, nullptr, &ctx), IRODORI_ERR_INVALID_ARG);
    irodori_dit_config g{};
    g.latent_dim = 32;
    g.model_dim = 256;
    g.num_layers = 2;
    g.num_heads = 4;
    g.head_dim = 64;
    g.mlp_hidden = 704;
    g.adaln_rank = 32;
    g.timestep_embed_dim = 64;
    g.norm_eps = 1e-6f;
    g.rope_theta = 10000.f;
    g.compute_dtype = IRODORI_DTYPE_BF16;
    g.max_rows = 2;
    g.max_seq = 64;
    g.max_ctx = 48;
    struct Bad {
        const char* what;
        void (*edit)(irodori_dit_config&);
        int code;
    } bad[] = {
        {"head_dim 96", [](irodori_dit_config& c) { c.head_dim = 96; }, IRODORI_ERR_SHAPE},
        {"latent 257", [](irodori_dit_config& c) { c.latent_dim = 257; }, IRODORI_ERR_SHAPE},
        {"dtype 9", [](irodori_dit_config& c) { c.compute_dtype = 9; }, IRODORI_ERR_DTYPE},
        {"eps 0", [](irodori_dit_config& c) { c.norm_eps = 0.f; }, IRODORI_ERR_CONFIG},
        {"rows 65536", [](irodori_dit_config& c) { c.max_rows = 65536; }, IRODORI_ERR_SHAPE},
        {"fp8 head 128",
         [](irodori_dit_config& c) {
             c.compute_dtype = IRODORI_DTYPE_FP8;
             c.num_heads = 2;
             c.head_dim = 128;
         },
         IRODORI_ERR_SHAPE},
        {"too many keys", [](irodori_dit_config& c) { c.max_seq = 16000; c.max_ctx = 1000; }, IRODORI_ERR_SHAPE},
    };
    for (const Bad& b : bad) {
        irodori_dit_config c = g;
        b.edit(c);
        ctx = nullptr;
        expect(b.what, irodori_ctx_create(0, &c, &ctx), b.code);
        if (ctx) failures++;
    }

    float dummy[16];
    expect("sdpa dtype", irodori_op_sdpa(7, dummy, dummy, dummy, nullptr, 1, 1, 1, 1, 64, 1.f, dummy, nullptr),
           IRODORI_ERR_DTYPE);
    expect("sdpa head_dim", irodori_op_sdpa(IRODORI_DTYPE_F32, dummy, dummy, dummy, nullptr, 1, 1, 1, 1, 96, 1.f, dummy,
                                            nullptr),
           IRODORI_ERR_SHAPE);
    expect("sdpa null", irodori_op_sdpa(IRODORI_DTYPE_BF16, nullptr, nullptr, nullptr, nullptr, 1, 1, 1, 1, 64, 1.f,
                                        nullptr, nullptr),
           IRODORI_ERR_INVALID_ARG);
    expect("forward null", irodori_forward(nullptr, 1, 1, nullptr, nullptr, nullptr, nullptr), IRODORI_ERR_INVALID_ARG);
    std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
    return failures ? 1 : 0;
}
