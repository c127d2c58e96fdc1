/*
 * sanitize_check.cpp -- host-side run of the oracle and of the library's
 * host code (argument checks, the weight store's archive and manifest
 * parsing) under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.
 *
 * Built by `make -C tests/native sanitize` (the sanitizers instrument the
 * host code of the library's sources; without a device no GPU launch path is
 * reached) and run by tests/test_sanitize.py with the VPK files it writes as
 * arguments.
 * Exits 0 when every check passes; a sanitizer report aborts the process.
 */
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "gemma4_sampler.h"
#include "../../oracle/g4s_oracle.h"

namespace {

int g_fail = 0;

#define CHECK(cond)                                                          \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
            ++g_fail;                                                        \
        }                                                                    \
    } while (0)

uint64_t g_state = 0x9E3779B97F4A7C15ull;

uint32_t next_u32()
{
    g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(g_state >> 32);
}

float next_normal(float sigma)
{
    /* sum of 12 uniforms: adequate spread for logits */
    float s = 0.0f;
    for (int i = 0; i < 12; ++i) s += (float)(next_u32() >> 8) * (1.0f / 16777216.0f);
    return (s - 6.0f) * sigma;
}

void oracle_checks()
{
    const int32_t vocabs[] = {1, 2, 3, 7, 64, 1000, 4099};
    const int32_t ks[] = {-1, 0, 1, 2, 63, 64, 1000, 5000};
    const float ts[] = {0.0f, 0.7f, 1.0f, -1.0f, 1.3f};
    const float ps[] = {0.0f, 0.5f, 0.95f, 1.0f};
    const float caps[] = {0.0f, 30.0f};
    for (int32_t V : vocabs) {
        std::vector<float> row((size_t)V);
        std::vector<int32_t> idx((size_t)V);
        std::vector<float> probs((size_t)V);
        for (int rep = 0; rep < 3; ++rep) {
            for (int32_t i = 0; i < V; ++i) {
                row[(size_t)i] = rep == 2 ? (float)(int)(next_u32() % 3) : next_normal(3.0f);
                if (rep == 1 && next_u32() % 5 == 0) row[(size_t)i] = -INFINITY;
            }
            for (int32_t K : ks)
                for (float T : ts)
                    for (float P : ps)
                        for (float cap : caps) {
                            orc_params p{T, K, P, 1.0f};
                            orc_detail d{};
                            const double u = (double)(next_u32()) / 4294967296.0;
                            const int32_t tok = orc_do_sample(row.data(), V, cap, &p, u, idx.data(),
                                                              probs.data(), V, &d);
                            CHECK(tok >= -1 && tok < V);
                        }
            for (int32_t K : ks) {
                if (K < 1) continue;
                const int32_t n = orc_select_topk_indices(row.data(), V, K < V ? K : V, idx.data());
                CHECK(n >= 0 && n <= K);
                for (int32_t i = 1; i < n; ++i) CHECK(idx[(size_t)i - 1] < idx[(size_t)i]);
            }
            std::vector<float> tmp = row;
            orc_logit_softcap(tmp.data(), V, 30.0f);
            (void)orc_softmax_f32(tmp.data(), V);
            int64_t first = -2;
            (void)orc_seqsum_f32(row.data(), V, 0.5f, &first);
            CHECK(first >= -1 && first < V);
        }
    }
    /* batches: fp32 and bf16, several threads */
    const int32_t V = 3000, B = 5;
    std::vector<float> rows((size_t)V * B);
    std::vector<uint16_t> rows16((size_t)V * B);
    for (size_t i = 0; i < rows.size(); ++i) {
        rows[i] = next_normal(2.0f);
        rows16[i] = orc_f32_to_bf16(rows[i]);
    }
    std::vector<orc_params> prm((size_t)B);
    std::vector<double> us((size_t)B);
    std::vector<int32_t> ids((size_t)B);
    for (int32_t b = 0; b < B; ++b) {
        prm[(size_t)b] = orc_params{0.7f, b == 0 ? 0 : 64, 0.95f, 1.0f};
        us[(size_t)b] = 0.25 * b;
    }
    CHECK(orc_sample_batch(rows.data(), 0, V, V, B, prm.data(), us.data(), 30.0f, ids.data(), 3) == 0);
    CHECK(orc_sample_batch(rows16.data(), 1, V, V, B, prm.data(), us.data(), 30.0f, ids.data(), 2) == 0);
    /* Q4_0 round trip and matvec */
    const int32_t rq = 70, cq = 96;
    std::vector<float> w((size_t)rq * cq), h((size_t)2 * cq), out((size_t)2 * rq);
    for (auto& x : w) x = next_normal(0.05f);
    for (auto& x : h) x = next_normal(1.0f);
    std::vector<uint8_t> q((size_t)rq * (cq / 32) * 18);
    CHECK(orc_f32_to_q4_buffer(w.data(), q.data(), w.size()) == q.size() / 18);
    float blk[32];
    orc_dequant_q4_block(q.data(), blk);
    orc_matvec_q4(q.data(), h.data(), out.data(), rq, cq, 3, rq - 3);
    orc_matvec_q4_batch(q.data(), h.data(), out.data(), rq, cq, 2, 3);
    for (uint32_t v = 0; v < 65536; v += 7) {
        (void)orc_f16_to_f32((uint16_t)v);
        (void)orc_bf16_to_f32((uint16_t)v);
    }
}

void library_checks()
{
    g4s_sampler* s = nullptr;
    const int rc = g4s_create(&s, 262144, 4, 30.0f, nullptr);
    CHECK(rc == G4S_ERR_NO_DEVICE || rc == G4S_OK);
    if (rc == G4S_OK) g4s_destroy(s);
    CHECK(std::strlen(g4s_last_error(nullptr)) < 512);
    CHECK(g4s_create(nullptr, 262144, 4, 30.0f, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    g4s_sampler* s2 = nullptr;
    CHECK(g4s_create(&s2, 1, 4, 30.0f, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_create(&s2, 262144, 0, 30.0f, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_create(&s2, 262144, 4, NAN, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    g4s_params p;
    g4s_params_set_defaults(&p);
    CHECK(p.top_k == 64);
    double u = 0.5;
    int32_t id = -7;
    CHECK(g4s_sample(nullptr, nullptr, 0, 1, 1, &p, &u, &id) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_sample_ex(nullptr, nullptr, 0, 1, 1, &p, &u, &id, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_sample_async(nullptr, nullptr, 0, 1, 1, nullptr, nullptr, 64, 0, nullptr, nullptr) ==
          G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_lmhead_q4_0(nullptr, nullptr, 1, 32, nullptr, 1, nullptr, 1) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_lmhead_q4_0_tiled(nullptr, nullptr, 1, 32, nullptr, 1, nullptr, 1) ==
          G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_lmhead_sample_q4_0(nullptr, nullptr, 32, nullptr, 1, nullptr, 1, &p, &u, &id,
                                 nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_embed_q4_0(nullptr, nullptr, 1, 32, nullptr, 1, 1.0f, nullptr) ==
          G4S_ERR_INVALID_ARGUMENT);
    int32_t toks[4], lens[1];
    CHECK(g4s_generate(nullptr, 1, &p, 4, nullptr, 0, 1, nullptr, nullptr, nullptr, nullptr, toks,
                       lens) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_q4_0_device_bytes(262144, 2560, G4S_Q4_LAYOUT_ROWS) == 377487360);
    CHECK(g4s_q4_0_device_bytes(65, 64, G4S_Q4_LAYOUT_TILED64) == 2 * 2 * 1280);
    CHECK(g4s_q4_0_device_bytes(0, 64, G4S_Q4_LAYOUT_ROWS) == -1);
    CHECK(g4s_q4_0_device_bytes(4, 40, G4S_Q4_LAYOUT_ROWS) == -1);
    CHECK(g4s_q4_0_repack(nullptr, 4, 32, nullptr, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_q4_0_repack((void*)16, 4, 40, (void*)32, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_sample_topk_noalloc(nullptr, 0, 262144, 262144, 1, nullptr, nullptr, 64, 30.0f,
                                  nullptr, nullptr, nullptr) != G4S_OK);
    CHECK(g4s_store_open(nullptr, "x", nullptr, nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_store_close(nullptr) == G4S_OK);
    CHECK(g4s_store_tensor_count(nullptr) == 0);
    CHECK(g4s_store_verify(nullptr) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_store_raw_pointer(nullptr, "x") == nullptr);
}

/* Every query of an archive that opened, and upload requests that fail
 * their checks before any device work. */
void store_checks(const char* path)
{
    g4s_store* st = nullptr;
    const int rc = g4s_store_open(&st, path, nullptr, nullptr);
    if (rc != G4S_OK) {
        CHECK(st == nullptr);
        CHECK(std::strlen(g4s_store_last_error(nullptr)) > 0);
        return;
    }
    const int32_t n = g4s_store_tensor_count(st);
    CHECK(n > 0);
    char name[1024];
    g4s_tensor_info info;
    CHECK(g4s_store_tensor_info(st, -1, &info, name, sizeof name) == G4S_ERR_INVALID_ARGUMENT);
    CHECK(g4s_store_tensor_info(st, n, &info, name, sizeof name) == G4S_ERR_INVALID_ARGUMENT);
    for (int32_t i = 0; i < n; ++i) {
        CHECK(g4s_store_tensor_info(st, i, &info, name, sizeof name) == G4S_OK);
        CHECK(g4s_store_tensor_info(st, i, nullptr, name, 1) != G4S_OK || name[0] == 0);
        g4s_tensor_info f;
        /* a name holding a NUL character is cut short in C and not found */
        const int fr = g4s_store_find_tensor(st, name, &f);
        CHECK(fr == G4S_OK || fr == G4S_ERR_NOT_FOUND);
        const void* raw = fr == G4S_OK ? g4s_store_raw_pointer(st, name) : nullptr;
        if (raw) {
            /* touch every byte of the tensor inside the mapping */
            const uint8_t* b = static_cast<const uint8_t*>(raw);
            uint32_t acc = 0;
            for (uint64_t j = 0; j < f.size; ++j) acc += b[j];
            (void)acc;
        }
        /* refused before any device work: unknown layout, a tiny buffer,
         * a misaligned one */
        CHECK(g4s_store_upload_q4_0(st, name, 9, (void*)4096, 1u << 20, nullptr) != G4S_OK);
        CHECK(g4s_store_upload_q4_0(st, name, 0, (void*)4096, 1, nullptr) != G4S_OK);
        CHECK(g4s_store_upload_q4_0(st, name, 0, (void*)4100, 1u << 30, nullptr) != G4S_OK);
    }
    CHECK(g4s_store_find_tensor(st, "no such tensor", &info) == G4S_ERR_NOT_FOUND);
    (void)g4s_store_verify(st);
    CHECK(g4s_store_close(st) == G4S_OK);
}

}  // namespace

int main(int argc, char** argv)
{
    oracle_checks();
    library_checks();
    for (int i = 1; i < argc; ++i) store_checks(argv[i]);
    if (g_fail) {
        std::fprintf(stderr, "%d checks failed\n", g_fail);
        return 1;
    }
    std::printf("sanitize_check: oracle, argument checks and %d archives clean\n", argc - 1);
    return 0;
}
