// Test infrastructure: drives every entry point of the CPU oracle
// (oracle/oracle.cpp, linked in) over random inputs, edge cases included, in
// a build with AddressSanitizer and UndefinedBehaviorSanitizer
// (locus_amd/build.py: build_sanitized). A sanitizer report fails the run;
// the few checks here are invariants (ids in range, survivors non-empty),
// since the oracle's values are pinned elsewhere.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

extern "C" {
struct orc_params {
    float temperature;
    uint32_t top_k;
    float top_p, min_p, repeat_penalty, frequency_penalty, presence_penalty;
    uint32_t repeat_last_n;
};
int32_t orc_sample(float* logits, uint32_t V, const orc_params* p, const int32_t* hist, uint32_t n_hist, double u,
                   const uint32_t* mask, void* diag);
void orc_logprobs(const float* logits, uint32_t V, int32_t chosen, uint32_t n_top, float* chosen_lp, int32_t* top_ids,
                  float* top_lp, uint32_t* tie);
int32_t orc_argmax(const float* logits, uint32_t V);
void orc_verify(const void* logits, int bf16, uint32_t n_seq, uint32_t rows_per_seq, uint32_t V, uint64_t row_stride,
                const int32_t* draft, int32_t* argmax_ids, float* draft_lp, uint32_t* accept_len, uint32_t threads);
void* orc_json_new(void);
void* orc_json_clone(const void* g);
void orc_json_free(void* g);
int orc_json_feed(void* g, uint8_t b);
int orc_json_complete(const void* g);
void orc_json_mask(const void* g, const uint8_t* blob, const uint64_t* off, uint32_t n_pieces, uint32_t V,
                   uint32_t* out);
uint32_t orc_ngram_draft(const int32_t* ctx, uint32_t n, uint32_t ngram, uint32_t max_draft, int32_t* out);
uint32_t orc_sizeof_diag(void);
double orc_mt_u(uint64_t seed, uint64_t skip);
}

static int g_fail = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            ++g_fail;                                                         \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #c); \
        }                                                                     \
    } while (0)

int main() {
    std::mt19937_64 g(77);
    std::normal_distribution<float> nd(0.0f, 2.0f);
    std::vector<unsigned char> diag(orc_sizeof_diag());
    for (int it = 0; it < 400; ++it) {
        const uint32_t V = 1 + static_cast<uint32_t>(g() % (it % 10 == 0 ? 3 : 3000));
        std::vector<float> l(V);
        const bool ints = it % 7 == 0;   // exact ties
        for (float& x : l) x = ints ? std::floor(nd(g)) : nd(g);
        orc_params p{};
        p.temperature = (it % 4 == 0) ? 0.0f : 0.2f + static_cast<float>(g() % 200) / 100.0f;
        p.top_k = (it % 3 == 0) ? static_cast<uint32_t>(g() % (V + 2)) : 0u;
        p.top_p = (it % 2 == 0) ? 0.5f + static_cast<float>(g() % 50) / 100.0f : 1.0f;
        p.min_p = (it % 5 == 0) ? static_cast<float>(g() % 30) / 100.0f : 0.0f;
        p.repeat_penalty = (it % 6 == 0) ? 1.3f : 1.0f;
        p.frequency_penalty = (it % 6 == 1) ? 0.4f : 0.0f;
        p.presence_penalty = (it % 6 == 2) ? 0.2f : 0.0f;
        p.repeat_last_n = static_cast<uint32_t>(g() % 100);
        std::vector<int32_t> hist(g() % 120);
        for (int32_t& t : hist) t = static_cast<int32_t>(g() % (V + 20)) - 10;   // negative and >= V ids too
        std::vector<uint32_t> mask((V + 31) / 32, 0);
        const bool masked = it % 3 == 1;
        if (masked)
            for (uint32_t t = 0; t < V; ++t)
                if (g() % 4 == 0 || it % 30 == 1) mask[t >> 5] |= 1u << (t & 31u);   // sometimes none allowed
        const double u = orc_mt_u(g(), 0);
        std::vector<float> row = l;
        const int32_t id = orc_sample(row.data(), V, &p, hist.data(), static_cast<uint32_t>(hist.size()), u,
                                      masked ? mask.data() : nullptr, diag.data());
        CHECK(id >= 0 && static_cast<uint32_t>(id) < V);
        const uint32_t n_top = static_cast<uint32_t>(g() % 25);
        std::vector<int32_t> ti(n_top + 1);
        std::vector<float> tl(n_top + 1);
        float clp = 1.0f;
        uint32_t tie = 0;
        orc_logprobs(l.data(), V, it % 11 == 0 ? -3 : id, n_top, &clp, ti.data(), tl.data(), &tie);
        CHECK(clp <= 0.0f);
        CHECK(orc_argmax(l.data(), V) >= 0);
    }
    {
        // verify, f32 and bf16 rows
        const uint32_t n_seq = 5, rps = 4, V = 777, S = 784;
        std::vector<float> f(static_cast<size_t>(n_seq) * rps * S);
        for (float& x : f) x = nd(g);
        std::vector<uint16_t> h(f.size());
        for (size_t i = 0; i < f.size(); ++i) {
            uint32_t b;
            std::memcpy(&b, &f[i], 4);
            h[i] = static_cast<uint16_t>(b >> 16);
        }
        std::vector<int32_t> draft(n_seq * rps), am(n_seq * rps);
        for (int32_t& d : draft) d = static_cast<int32_t>(g() % (V + 4)) - 2;
        std::vector<float> dlp(n_seq * rps);
        std::vector<uint32_t> acc(n_seq);
        orc_verify(f.data(), 0, n_seq, rps, V, S, draft.data(), am.data(), dlp.data(), acc.data(), 2);
        for (uint32_t a : acc) CHECK(a <= rps);
        orc_verify(h.data(), 1, n_seq, rps, V, S, draft.data(), am.data(), dlp.data(), acc.data(), 1);
        for (uint32_t a : acc) CHECK(a <= rps);
    }
    {
        // grammar: random bytes, clones, masks over random pieces
        std::vector<uint8_t> blob;
        std::vector<uint64_t> off{0};
        const char alpha[] = "{}[]\",:0123456789.-+eEtrufalsn \\/u";
        for (int k = 0; k < 300; ++k) {
            const int n = static_cast<int>(g() % 6);
            for (int j = 0; j < n; ++j) blob.push_back(static_cast<uint8_t>(alpha[g() % (sizeof(alpha) - 1)]));
            off.push_back(blob.size());
        }
        std::vector<uint32_t> out((310 + 31) / 32);
        for (int it = 0; it < 200; ++it) {
            void* j = orc_json_new();
            for (int k = 0; k < 40; ++k) {
                if (!orc_json_feed(j, static_cast<uint8_t>(alpha[g() % (sizeof(alpha) - 1)]))) break;
                if (k % 8 == 0) orc_json_mask(j, blob.data(), off.data(), 300, 310, out.data());
            }
            void* c = orc_json_clone(j);
            (void)orc_json_complete(c);
            orc_json_free(c);
            orc_json_free(j);
        }
    }
    {
        std::vector<int32_t> out(8);
        for (int it = 0; it < 500; ++it) {
            std::vector<int32_t> ctx(g() % 20);
            for (int32_t& t : ctx) t = static_cast<int32_t>(g() % 3);
            const uint32_t n = orc_ngram_draft(ctx.data(), static_cast<uint32_t>(ctx.size()),
                                               static_cast<uint32_t>(g() % 4), static_cast<uint32_t>(g() % 9),
                                               out.data());
            CHECK(n <= 8);
        }
    }
    std::printf("oracle_asan: %d failures\n", g_fail);
    return g_fail == 0 ? 0 : 1;
}
