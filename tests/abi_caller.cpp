// A C++ program that binds libjxmoe.so through include/jxmoe.h alone, the way
// the reference engine would (the binding of bind_tensors and the forward of
// MoETransformerEngine::forward_token, src/transformer.cpp:2142-2186 and
// 2589-2764): init, create a layer from packed GGUF-layout expert tensors,
// run the MoE block for one token and for a batch, add the residual.
//
//   abi_caller nodevice          expects jx_moe_init to fail with JX_ERR_NODEVICE
//   abi_caller run <dir>         writes the seeded layer, tokens and results to <dir>
//
// The layer is Q4_0, d_model 512, 8 experts, top-2, d_ff 1024, generated from a
// fixed 64-bit LCG so the test that runs this program can rebuild the same
// layer through the Python binding and compare results bit for bit.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "jxmoe.h"

namespace {

struct Lcg {
    uint64_t s;
    uint32_t next() {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return (uint32_t)(s >> 33);
    }
    float unit() { return (next() & 0xFFFFFF) / 16777216.0f; }  // [0, 1)
};

// fp16 bits of a value in [2^-14, 65504] (round toward zero is enough for seeded scales)
uint16_t to_f16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t e = ((u >> 23) & 0xFF) - 112, m = (u & 0x7FFFFF) >> 13;
    return (uint16_t)((e << 10) | m);
}

// rows x cols Q4_0 blocks (18 bytes per 32 values: fp16 d, 16 bytes of nibbles)
std::vector<uint8_t> q4_0_matrix(Lcg& g, size_t rows, size_t cols) {
    std::vector<uint8_t> w(rows * (cols / 32) * 18);
    for (size_t b = 0; b < w.size() / 18; ++b) {
        const uint16_t d = to_f16(0.005f + 0.015f * g.unit());
        std::memcpy(&w[b * 18], &d, 2);
        for (int i = 0; i < 16; ++i) w[b * 18 + 2 + i] = (uint8_t)g.next();
    }
    return w;
}

bool dump(const std::string& path, const void* p, size_t n) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(p, 1, n, f) == n;
    return std::fclose(f) == 0 && ok;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "nodevice") == 0) {
        const int rc = jx_moe_init(0);
        std::printf("jx_moe_init -> %d (%s)\n", rc, jx_moe_last_error());
        jx_moe_layer* L = nullptr;
        jx_moe_layer_desc d{};
        const int rc2 = jx_moe_layer_create(&d, &L);
        std::printf("jx_moe_layer_create before init -> %d\n", rc2);
        return (rc == JX_ERR_NODEVICE && rc2 == JX_ERR_NODEVICE && L == nullptr) ? 0 : 1;
    }
    if (argc < 3 || std::strcmp(argv[1], "run") != 0) {
        std::fprintf(stderr, "usage: abi_caller nodevice | run <dir>\n");
        return 2;
    }
    const std::string dir = argv[2];
    const int E = 8, K = 2, D = 512, FF = 1024, NB = 64;
    Lcg g{20261201};
    std::vector<float> router((size_t)E * D);
    for (float& v : router) v = 0.04f * (g.unit() - 0.5f);
    const auto gate = q4_0_matrix(g, (size_t)E * FF, D);
    const auto up = q4_0_matrix(g, (size_t)E * FF, D);
    const auto down = q4_0_matrix(g, (size_t)E * D, FF);
    std::vector<float> x((size_t)NB * D);
    for (float& v : x) v = 4.0f * (g.unit() - 0.5f);

    // load_model: init once, then one layer from its expert tensors
    if (jx_moe_init(0) != JX_OK) {
        std::fprintf(stderr, "jx_moe_init: %s\n", jx_moe_last_error());
        return 1;
    }
    jx_moe_layer_desc d{};
    d.n_experts = E;
    d.top_k = K;
    d.d_model = D;
    d.d_ff = FF;
    d.gate_type = d.up_type = d.down_type = JX_TYPE_Q4_0;
    d.router = router.data();
    d.gate_exps = gate.data();
    d.up_exps = up.data();
    d.down_exps = down.data();
    jx_moe_layer* layer = nullptr;
    if (jx_moe_layer_create(&d, &layer) != JX_OK) {
        std::fprintf(stderr, "jx_moe_layer_create: %s\n", jx_moe_last_error());
        return 1;
    }
    // forward_token: the MoE block of one token, then the residual add (transformer.cpp:2762-2764)
    std::vector<int32_t> ids1(K);
    std::vector<float> probs1(K), accum1(D), resid(x.begin(), x.begin() + D);
    if (jx_moe_forward(layer, x.data(), 1, accum1.data(), ids1.data(), probs1.data(), nullptr, nullptr, 0) != JX_OK) {
        std::fprintf(stderr, "jx_moe_forward: %s\n", jx_moe_last_error());
        return 1;
    }
    for (int i = 0; i < D; ++i) resid[i] += accum1[i];
    // a prompt of NB tokens in one call (the matrix-core regime)
    std::vector<int32_t> ids((size_t)NB * K), counts(E);
    std::vector<float> probs((size_t)NB * K), out((size_t)NB * D);
    if (jx_moe_forward(layer, x.data(), NB, out.data(), ids.data(), probs.data(), counts.data(), nullptr, 0) !=
        JX_OK) {
        std::fprintf(stderr, "jx_moe_forward: %s\n", jx_moe_last_error());
        return 1;
    }
    jx_moe_layer_destroy(layer);
    bool ok = dump(dir + "/router.bin", router.data(), router.size() * 4) && dump(dir + "/gate.bin", gate.data(), gate.size()) &&
              dump(dir + "/up.bin", up.data(), up.size()) && dump(dir + "/down.bin", down.data(), down.size()) &&
              dump(dir + "/x.bin", x.data(), x.size() * 4) && dump(dir + "/out1.bin", accum1.data(), accum1.size() * 4) &&
              dump(dir + "/resid1.bin", resid.data(), resid.size() * 4) &&
              dump(dir + "/ids1.bin", ids1.data(), ids1.size() * 4) && dump(dir + "/out.bin", out.data(), out.size() * 4) &&
              dump(dir + "/ids.bin", ids.data(), ids.size() * 4) && dump(dir + "/counts.bin", counts.data(), counts.size() * 4);
    std::printf("token 0 experts %d %d, counts", ids1[0], ids1[1]);
    for (int e = 0; e < E; ++e) std::printf(" %d", counts[e]);
    std::printf("\n");
    return ok ? 0 : 1;
}
