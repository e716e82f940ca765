// Host-side fuzz of the C ABI under AddressSanitizer / UndefinedBehaviorSanitizer
// (built by tests/sanitize/Makefile; no GPU needed).  Random parameter structs
// -- valid ones, single-field mutations and absurd values -- go through every
// validation, workspace query and entry point with null tensor pointers, so
// each call returns a status before any HIP call; the sanitizers report any
// out-of-bounds access, signed overflow or other undefined behaviour on the
// way (the reference's contract test, tests/fused_bwd_api_contract.cpp:34-118,
// checks the statuses of the same paths).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "shaobo_fa3_api.h"
#include "shaobo_fa3_components.h"
#include "shaobo_fa3_ext.h"

namespace {

std::mt19937_64 rng(20261202);

int32_t pick_int() {
    static const int32_t edge[] = {0,  1,   -1,  2,    7,    64,         96,        128,
                                   256, 1000, 4096, 65536, 1 << 20, 0x7FFFFFFF, INT32_MIN};
    if (rng() % 3 == 0) return (int32_t)rng();
    return edge[rng() % (sizeof(edge) / sizeof(edge[0]))];
}

void random_params(ShaoboFa3Params* p) {
    shaobo_fa3_params_init(p);
    const int mode = (int)(rng() % 3);
    if (mode == 0) {  // a valid-looking shape
        p->batch = 1 + (int)(rng() % 4);
        p->num_heads_kv = 1 + (int)(rng() % 4);
        p->num_heads_q = p->num_heads_kv * (1 + (int)(rng() % 4));
        p->seqlen_q = p->seqlen_k = 128 * (1 + (int)(rng() % 32));
        p->head_dim_qk = p->head_dim_v = (rng() & 1) ? 64 : 128;
        p->causal = (int)(rng() % 2);
        p->softmax_scale = 0.125f;
        p->dtype = (int)(rng() % 2);
        p->layout = (int)(rng() % 2);
    }
    // mutate a few fields, sometimes to absurd values
    const int n = mode == 0 ? (int)(rng() % 3) : 4 + (int)(rng() % 12);
    for (int i = 0; i < n; ++i) {
        switch (rng() % 16) {
            case 0: p->batch = pick_int(); break;
            case 1: p->seqlen_q = pick_int(); break;
            case 2: p->seqlen_k = pick_int(); break;
            case 3: p->num_heads_q = pick_int(); break;
            case 4: p->num_heads_kv = pick_int(); break;
            case 5: p->head_dim_qk = pick_int(); break;
            case 6: p->head_dim_v = pick_int(); break;
            case 7: p->causal = pick_int(); break;
            case 8: p->window_left = pick_int(); p->window_right = pick_int(); break;
            case 9: p->dtype = pick_int(); break;
            case 10: p->layout = pick_int(); break;
            case 11: p->softmax_aux_mode = pick_int(); break;
            case 12: p->dkv_path = pick_int(); p->dq_path = pick_int(); break;
            case 13: p->deterministic = pick_int(); break;
            case 14: p->struct_size = (uint32_t)pick_int(); break;
            default: p->dropout_p = (rng() & 1) ? 0.1f : 0.f; break;
        }
    }
    if (rng() % 4 == 0) p->dkv_path = 1;
    if (rng() % 4 == 0) p->dq_path = 1;
    p->workspace = nullptr;
    p->workspace_bytes = rng() % 2 ? 0 : ~(size_t)0;
}

}  // namespace

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
    size_t sink = 0;
    int statuses[8] = {};
    ShaoboFa3Params p;
    for (int it = 0; it < iters; ++it) {
        random_params(&p);
        int st = shaobo_fa3_bwd_v2_validate(&p);
        statuses[st & 7]++;
        sink += shaobo_fa3_bwd_v2_workspace_bytes(&p);
        sink += shaobo_fa3_bwd_workspace_bytes(&p);
        sink += shaobo_fa3_bwd_fused5_workspace_bytes(&p);
        sink += shaobo_fa3_bwd_dkv_workspace_bytes(&p);
        sink += shaobo_fa3_bwd_dq_workspace_bytes(&p);
        void* n = nullptr;
        // every tensor pointer null: each entry returns before launching
        sink += shaobo_fa3_bwd_v2(n, n, n, n, n, n, n, n, n, n, &p);
        sink += shaobo_fa3_bwd_v2_on_stream(n, n, n, n, n, n, n, n, n, n, &p, n);
        sink += shaobo_fa3_ext_bwd_v2_no_alloc(n, n, n, n, n, n, n, n, n, n, &p, n);
        sink += shaobo_fa3_ext_bwd_v2_timed(n, n, n, n, n, n, n, n, n, n, &p, n, nullptr);
        sink += shaobo_fa3_bwd(n, n, n, n, n, n, n, n, n, n, &p);
        sink += shaobo_fa3_bwd_dot_do_o(n, n, n, n, n, n, &p);
        sink += shaobo_fa3_bwd_fused5(n, n, n, n, n, n, n, n, &p);
        sink += shaobo_fa3_bwd_dkv(n, n, n, n, n, n, n, n, n, n, &p);
        sink += shaobo_fa3_bwd_dq(n, n, n, n, n, n, n, n, n, n, &p);
        sink += std::strlen(shaobo_fa3_status_string(pick_int()));
    }
    // null params everywhere
    sink += shaobo_fa3_bwd_v2_validate(nullptr) + shaobo_fa3_bwd_v2_workspace_bytes(nullptr);
    sink += shaobo_fa3_bwd_workspace_bytes(nullptr) + shaobo_fa3_bwd_fused5_workspace_bytes(nullptr);
    sink += shaobo_fa3_bwd_dkv_workspace_bytes(nullptr) + shaobo_fa3_bwd_dq_workspace_bytes(nullptr);
    ShaoboFa3BwdCapabilities caps;
    std::memset(&caps, 0, sizeof(caps));
    sink += shaobo_fa3_bwd_get_capabilities(nullptr) + shaobo_fa3_bwd_get_capabilities(&caps);
    caps.struct_size = sizeof(caps);
    sink += shaobo_fa3_bwd_get_capabilities(&caps);
    std::printf("abi_fuzz: %d structs, validate statuses %d/%d/%d/%d/%d, checksum %zu\n", iters,
                statuses[0], statuses[1], statuses[2], statuses[3], statuses[4], sink);
    return 0;
}
