// Host-layer tests in C++ against the public headers (include/locus/...):
// the reference's own known-answer tests for sampling, the JSON grammar and
// the n-gram draft (tests/test_sampling.cpp, test_grammar.cpp,
// test_speculative.cpp), restated with a minimal harness, plus the mask
// builder against per-token allows() and the backend-resolution rules.
//   test_host cpu   grammar, mask builder, n-gram draft, registry (no device)
//   test_host gpu   sampling API on the device, registry with a device, and
//                   the batched engine step against the per-row API
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include "locus/backend/sampler_registry.hpp"
#include "locus/engine/batch_sampler.hpp"
#include "locus/model/grammar.hpp"
#include "locus/model/sampling.hpp"
#include "locus/model/speculative.hpp"

using namespace locus::model;
using locus::tok::TokenId;

static int g_fail = 0, g_pass = 0;
#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (cond) {                                                                   \
            ++g_pass;                                                                 \
        } else {                                                                      \
            ++g_fail;                                                                 \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);      \
        }                                                                             \
    } while (0)

template <class E, class F>
static bool throws(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

static bool feed_all(JsonGrammar& g, const std::string& s) {
    for (unsigned char c : s)
        if (!g.feed(c)) return false;
    return true;
}

static void test_grammar() {
    for (const char* s : {"{}", "[]", "\"hi\"", "123", "-1.5e3", "true", "false", "null", "{\"a\":1}",
                          "[1,2,3]", "{\"a\":[1,{\"b\":\"c\"}],\"d\":null}", "  {  \"x\" : 1 }  ",
                          "[ -0.5 , 2 ]", "[12,34]", "{\"n\":42}", "42", "42   ", "\"\\u00e9\\n\""}) {
        JsonGrammar g;
        const bool ok = feed_all(g, s) && g.complete();
        if (!ok) std::fprintf(stderr, "  accept: %s\n", s);
        CHECK(ok);
    }
    for (const char* s : {"{", "{\"a\"", "{\"a\":", "[1,", "\"ab", "tr", "-", "[1"}) {
        JsonGrammar g;
        CHECK(feed_all(g, s));
        CHECK(!g.complete());
    }
    for (const char* s : {"{,}", "[,]", "[1,]", "{\"a\" 1}", "{1:2}", "trux", "{}x", "01a", "[1 2]", "}",
                          "42x", "\"\\x\"", "\"\\u12g\"", "[}", "{]"}) {
        JsonGrammar g;
        const bool rej = !feed_all(g, s);
        if (!rej) std::fprintf(stderr, "  reject: %s\n", s);
        CHECK(rej);
    }
    JsonGrammar g;
    CHECK(feed_all(g, "{}"));
    CHECK(g.complete());
    CHECK(g.feed(' '));
    CHECK(g.complete());
    CHECK(!g.feed('x'));
}

static std::vector<std::string> synthetic_pieces() {
    std::vector<std::string> p;
    for (int b = 0; b < 256; ++b) p.push_back(std::string(1, static_cast<char>(b)));
    for (const char* s : {"{\"", "\":", "\", \"", "\"}", "true", "false", "null", "tru", "ul", "123", "-0.5e3",
                          "1.", "e+", "\\u00", "e9", "\\n", "  ", "\n  ", "},", "]}", "[[", "]]", "{}", "[]",
                          ",\"", "\": \"", "\":[", "\":{", "abc", "ab\"", "\"a\":1", "1,2", "0]", "}}", "\"\"",
                          "x", "", ""}) {
        p.push_back(s);
    }
    std::mt19937_64 r(7);
    const char alpha[] = "{}[]\":,. -+eE0123456789tfnrulsa\\bx \n";
    for (int i = 0; i < 600; ++i) {
        std::string s;
        const int n = 1 + static_cast<int>(r() % 12);
        for (int k = 0; k < n; ++k) s.push_back(alpha[r() % (sizeof(alpha) - 1)]);
        p.push_back(s);
    }
    return p;
}

static void test_mask_builder() {
    auto pieces = synthetic_pieces();
    auto mb = std::make_shared<const JsonMaskBuilder>(pieces, 64);
    const std::uint32_t V = static_cast<std::uint32_t>(pieces.size()) + 37;   // tail tokens allowed
    const std::uint32_t words = (V + 31) / 32;
    std::vector<std::uint32_t> m(words), brute(words);
    int states = 0, mism = 0;
    for (const char* doc : {"{\"a\": [1, -2.5e3, true, null, {\"b\": \"x\\u00e9y\\n\"}], \"c\": false}",
                            "[[[[{\"k\":[]}]]], \"s\", 0]", "  \"str\"  ", "-12.5E+3", "{\"a\":{\"b\":{\"c\":{}}}}"}) {
        JsonTokenConstraint c(mb);
        const std::string d = doc;
        for (std::size_t i = 0; i <= d.size(); ++i) {
            CHECK(c.allow_mask(V, m.data()));
            std::fill(brute.begin(), brute.end(), 0u);
            for (std::uint32_t t = 0; t < V; ++t)
                if (c.allows(static_cast<TokenId>(t))) brute[t >> 5] |= 1u << (t & 31);
            ++states;
            if (m != brute) ++mism;
            // a second build of the same state comes from the cache and must agree
            std::vector<std::uint32_t> again(words);
            c.allow_mask(V, again.data());
            if (again != m) ++mism;
            if (i < d.size()) {
                // advance by the single-byte token of the next byte (piece t == byte t)
                c.commit(static_cast<TokenId>(static_cast<unsigned char>(d[i])));
            }
        }
    }
    std::fprintf(stderr, "  mask builder: %d states, %d mismatches, cache hits/misses %llu/%llu\n", states,
                 mism, (unsigned long long)mb->cache_stats().first, (unsigned long long)mb->cache_stats().second);
    CHECK(states > 100);
    CHECK(mism == 0);
}

static void test_ngram() {
    CHECK((ngram_draft(std::vector<TokenId>{1, 2, 3, 4, 1, 2, 3}, 2, 3) == std::vector<TokenId>{4, 1, 2}));
    CHECK((ngram_draft(std::vector<TokenId>{9, 9, 5, 9, 9, 7, 9, 9}, 2, 2) == std::vector<TokenId>{7, 9}));
    const std::vector<TokenId> none{5, 6, 7}, tiny{1, 2};
    CHECK(ngram_draft(none, 2, 3).empty());
    CHECK(ngram_draft(tiny, 2, 3).empty());
    CHECK(ngram_draft(none, 0, 3).empty());
    CHECK(ngram_draft(none, 1, 0).empty());
    // overlapping match: the draft may run into the trailing n-gram itself
    CHECK((ngram_draft(std::vector<TokenId>{3, 3, 3}, 1, 5) == std::vector<TokenId>{3}));
}

// A stand-in for the application's CPU sampler (the integration registers the
// reference's own sample()/logprobs_from() this way): greedy on the first max.
static TokenId first_max(std::span<float> l, const SamplingParams&, std::span<const TokenId>, std::mt19937_64&,
                         const TokenConstraint*) {
    std::size_t best = 0;
    for (std::size_t i = 1; i < l.size(); ++i)
        if (l[i] > l[best]) best = i;
    return static_cast<TokenId>(best);
}

static void test_registry(bool gpu) {
    using namespace locus::backend;
    {
        const auto all = sampler_backends();
        CHECK(all.size() == 1 && all[0].name == "hip");
        CHECK(all[0].ops.sample_batch != nullptr && all[0].ops.sample != nullptr);
    }
    CHECK(find_sampler_backend("hip") != nullptr);
    CHECK(find_sampler_backend("scalar") == nullptr);
    CHECK(throws<std::invalid_argument>([] { resolve_sampler_backend("scalar"); }));
    CHECK(throws<std::invalid_argument>([] { resolve_sampler_backend("bogus"); }));
    if (gpu) {
        CHECK(sampler_backends()[0].available);
        CHECK(resolve_sampler_backend("").name == "hip");
        CHECK(resolve_sampler_backend("hip").name == "hip");
        CHECK(best_sampler_backend().ops.sample_batch != nullptr);
    } else {
        CHECK(!sampler_backends()[0].available);
        CHECK(throws<std::runtime_error>([] { best_sampler_backend(); }));
        CHECK(throws<std::invalid_argument>([] { resolve_sampler_backend("hip"); }));
    }
    // the fallback hook: after the application registers its CPU sampler,
    // best_sampler_backend() never throws (registry.cpp:105-111)
    const auto before = sampler_backends();
    SamplerOps ops;
    ops.sample = &first_max;
    CHECK(register_sampler_backend({"scalar", "application CPU sampler", true, true, ops}));
    CHECK(!register_sampler_backend({"scalar", "a second one", true, true, ops}));   // name taken
    CHECK(!register_sampler_backend({"hip", "shadow", true, true, ops}));
    CHECK(before.size() == 1 && before[0].name == "hip");   // earlier spans stay valid
    CHECK(sampler_backends().size() == 2 && sampler_backends()[1].name == "scalar");
    CHECK(resolve_sampler_backend("scalar").ops.sample == &first_max);
    const SamplerBackend& best = best_sampler_backend();
    CHECK(best.name == (gpu ? "hip" : "scalar"));
    std::vector<float> l{1.0f, 3.0f, 2.0f};
    std::mt19937_64 rng(1);
    CHECK(best.ops.sample(l, SamplingParams{}, {}, rng, nullptr) == 1);
    CHECK(&resolve_sampler_backend("") == &best);
    ::setenv("LOCUS_SAMPLER_BACKEND", "scalar", 1);
    CHECK(resolve_sampler_backend("").name == "scalar");
    ::setenv("LOCUS_SAMPLER_BACKEND", "bogus", 1);
    CHECK(throws<std::invalid_argument>([] { resolve_sampler_backend(""); }));
    ::unsetenv("LOCUS_SAMPLER_BACKEND");
}

namespace {
struct AllowSet : TokenConstraint {
    std::set<TokenId> ok;
    bool allows(TokenId t) const override { return ok.count(t) > 0; }
    void commit(TokenId) override {}
};
}  // namespace

static void test_sampling_gpu() {
    std::mt19937_64 rng(123);
    const std::vector<TokenId> none;
    {
        std::vector<float> l{1.0f, 3.0f, 2.0f, 0.5f};
        CHECK(sample(l, SamplingParams{}, none, rng) == 1);
    }
    {
        std::vector<float> l{5.0f, 4.9f};
        SamplingParams p;
        p.repeat_penalty = 10.0f;
        const std::vector<TokenId> h{0};
        CHECK(sample(l, p, h, rng) == 1);
        CHECK(l[0] == 0.5f);   // penalised in place
    }
    {
        std::vector<float> l{5.0f, 4.0f};
        SamplingParams p;
        p.frequency_penalty = 1.0f;
        const std::vector<TokenId> h{0, 0, 0};
        CHECK(sample(l, p, h, rng) == 1);
        CHECK(l[0] == 2.0f);
    }
    {
        SamplingParams p;
        p.temperature = 1.5f;
        p.top_k = 1;
        for (int i = 0; i < 20; ++i) {
            std::vector<float> l{0.1f, 0.2f, 5.0f, 0.3f};
            CHECK(sample(l, p, none, rng) == 2);
        }
    }
    {
        SamplingParams p;
        p.temperature = 1.0f;
        std::mt19937_64 a(42), b(42);
        for (int i = 0; i < 16; ++i) {
            std::vector<float> la{1, 1, 1, 1}, lb{1, 1, 1, 1};
            CHECK(sample(la, p, none, a) == sample(lb, p, none, b));
        }
        // exactly one engine output per stochastic call, none per greedy call
        std::mt19937_64 c(42), d(42);
        std::vector<float> l{1, 2, 3};
        sample(l, p, none, c);
        d();
        CHECK(c() == d());
        std::vector<float> g{1, 2, 3};
        sample(g, SamplingParams{}, none, c);
        CHECK(c() == d());
    }
    {
        AllowSet c;
        c.ok = {2, 3};
        std::vector<float> l{5.0f, 4.0f, 3.0f, 2.0f, 1.0f};
        CHECK(sample(l, SamplingParams{}, none, rng, &c) == 2);
        SamplingParams p;
        p.temperature = 1.0f;
        for (int i = 0; i < 30; ++i) {
            std::vector<float> m{5.0f, 4.0f, 3.0f, 2.0f, 1.0f};
            CHECK(c.ok.count(sample(m, p, none, rng, &c)) == 1);
        }
    }
    {
        SamplingParams p;
        p.temperature = 1.0f;
        for (int i = 0; i < 50; ++i) {
            std::vector<float> l{0.0f, 40.0f, 0.0f};
            CHECK(sample(l, p, none, rng) == 1);
        }
    }
    {
        const std::vector<float> l{1.0f, 2.0f, 3.0f};
        float clp = 0.0f;
        std::vector<TokenLogprob> top;
        logprobs_from(l, 2, 3, clp, top);
        double psum = 0.0;
        for (const auto& t : top) psum += std::exp(static_cast<double>(t.logprob));
        CHECK(std::fabs(psum - 1.0) < 1e-5);
        CHECK(top.size() == 3 && top[0].token == 2 && top[1].token == 1 && top[2].token == 0);
        CHECK(std::fabs(top[0].logprob - clp) < 1e-6);
        for (const auto& t : top) CHECK(t.logprob <= 0.0f);
        std::vector<TokenLogprob> one;
        float lp2 = 0.0f;
        logprobs_from(l, 0, 1, lp2, one);
        CHECK(one.size() == 1 && one[0].token == 2);
        CHECK(lp2 < clp);
        float lp3 = 1.0f;
        logprobs_from(l, 7, 0, lp3, one);   // chosen outside [0, V): 0
        CHECK(lp3 == 0.0f && one.empty());
    }
    {
        std::vector<float> l{0.5f, 2.0f, -1.0f, 2.0f};
        CHECK(sample(l, SamplingParams{}, none, rng) == 1);   // greedy: first index of the max
    }
    {
        // JSON mask through allow_mask(): a sampled row only draws allowed tokens
        std::vector<std::string> pieces{"{", "}", "\"", "a", ":", "1", ",", " ", "x", "]"};
        auto mb = std::make_shared<const JsonMaskBuilder>(pieces);
        JsonTokenConstraint c(mb);
        SamplingParams p;
        p.temperature = 1.0f;
        std::string out;
        for (int step = 0; step < 6; ++step) {
            std::vector<float> l(12, 0.0f);
            const TokenId t = sample(l, p, none, rng, &c);
            CHECK(c.allows(t));
            c.commit(t);
            if (t < 10) out += pieces[t];
        }
        JsonGrammar g;
        CHECK(feed_all(g, out));
    }
}

// The CPU oracle (oracle/liboracle.so, test infrastructure): the reference's
// sample() and logprobs_from() restated, loaded from the tree next to this
// program as the checker.
namespace {
struct OracleParams {   // orc_params == SamplingParams, field for field
    float temperature;
    std::uint32_t top_k;
    float top_p, min_p, repeat_penalty, frequency_penalty, presence_penalty;
    std::uint32_t repeat_last_n;
};
using OrcSample = std::int32_t (*)(float*, std::uint32_t, const OracleParams*, const std::int32_t*, std::uint32_t,
                                   double, const std::uint32_t*, void*);
using OrcLogprobs = void (*)(const float*, std::uint32_t, std::int32_t, std::uint32_t, float*, std::int32_t*, float*,
                             std::uint32_t*);
struct Oracle {
    OrcSample sample = nullptr;
    OrcLogprobs logprobs = nullptr;
};
Oracle load_oracle() {
    char exe[4096] = {0};
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    std::string dir = n > 0 ? std::string(exe, static_cast<std::size_t>(n)) : std::string("tests/cpp/test_host");
    dir = dir.substr(0, dir.rfind('/'));
    const std::string path = dir + "/../../oracle/liboracle.so";
    void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!h) throw std::runtime_error("the oracle is not built: " + path);
    Oracle o;
    o.sample = reinterpret_cast<OrcSample>(dlsym(h, "orc_sample"));
    o.logprobs = reinterpret_cast<OrcLogprobs>(dlsym(h, "orc_logprobs"));
    if (!o.sample || !o.logprobs) throw std::runtime_error("oracle symbols missing");
    return o;
}
}  // namespace

// BatchSampler (one lcs_sample per step) against two twins driven the way
// Engine::sample_from drives a request (engine.cpp:423-450), each with its own
// copy of the requests (same seeds, histories, constraint states):
//   b: the per-row API (sample()/logprobs_from() on the device);
//   c: the CPU oracle (the reference's sample()/logprobs_from() restated),
//      with u drawn from the request's mt19937_64 as the reference draws it
//      and the constraint's allow words as its candidate filter.
// Ids, histories, constraint states and RNG positions must agree step by
// step, logprobs within 1e-5. The per-row API runs the exact path (it writes
// the penalised logits back), the batch the sliced paths, so this also
// checks the paths against each other.
static void test_batch_gpu() {
    using locus::engine::BatchSampler;
    using locus::sampler::SampleRequest;
    constexpr std::uint32_t V = 5003, B = 8, K = 5, STRIDE = (V + 3) / 4 * 4;
    std::vector<std::string> pieces = synthetic_pieces();
    std::mt19937_64 pr(11);
    const char alpha[] = "{}[]\":,. -+eE0123456789tfnrulsa\\bx \n";
    while (pieces.size() < V) {
        std::string t;
        const int n = 1 + static_cast<int>(pr() % 6);
        for (int k = 0; k < n; ++k) t.push_back(alpha[pr() % (sizeof(alpha) - 1)]);
        pieces.push_back(t);
    }
    auto mb = std::make_shared<const JsonMaskBuilder>(pieces);
    JsonTokenConstraint ca(mb), cb(mb), cc(mb);
    const Oracle orc = load_oracle();
    std::vector<SampleRequest> a(B), b(B), c(B);
    for (std::uint32_t r = 0; r < B; ++r) {
        SamplingParams& p = a[r].sampling;
        switch (r) {
            case 0: break;   // greedy
            case 1: p.temperature = 0.8f; p.top_k = 40; p.top_p = 0.95f; break;
            case 2: p.temperature = 0.7f; p.min_p = 0.05f; p.top_p = 0.9f; p.repeat_penalty = 1.1f;
                    p.frequency_penalty = 0.5f; p.presence_penalty = 0.3f; p.repeat_last_n = 2048; break;
            case 3: p.temperature = 1.5f; p.top_p = 0.98f; break;
            case 4: p.temperature = 1.0f; p.top_p = 0.95f; break;   // JSON constraint
            case 5: p.temperature = 1.0f; p.repeat_penalty = 1.3f; break;
            case 6: p.repeat_penalty = 1.2f; p.presence_penalty = 0.5f; break;   // greedy, penalties
            default: p.temperature = 0.9f; p.top_k = 100; break;   // exact path in both
        }
        a[r].rng.seed(1000 + r);
        for (int i = 0; i < 30; ++i) a[r].generated.push_back(static_cast<TokenId>(pr() % V));
        if (r == 1 || r == 2 || r == 6) a[r].logprobs_opt = {true, r == 1 ? 5u : (r == 2 ? 3u : 1u)};
        b[r] = a[r];
        c[r] = a[r];
    }
    a[4].constraint = &ca;
    b[4].constraint = &cb;
    c[4].constraint = &cc;
    std::vector<std::uint32_t> words((V + 31) / 32);
    std::vector<SampleRequest*> ap(B);
    for (std::uint32_t r = 0; r < B; ++r) ap[r] = &a[r];
    BatchSampler bs(0, B, V, 4096, 20);
    float* dlog = nullptr;
    CHECK(hipMalloc(&dlog, (std::size_t)B * STRIDE * sizeof(float)) == hipSuccess);
    std::mt19937 lr(99);
    std::normal_distribution<float> nd(0.0f, 2.0f);
    std::vector<float> host((std::size_t)B * STRIDE, 0.0f);
    for (std::uint32_t step = 0; step < K; ++step) {
        for (std::uint32_t r = 0; r < B; ++r)
            for (std::uint32_t i = 0; i < V; ++i) host[(std::size_t)r * STRIDE + i] = nd(lr);
        CHECK(hipMemcpy(dlog, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice) == hipSuccess);
        const std::vector<TokenId> ids = bs.sample_step(dlog, LCS_F32, STRIDE, ap);
        CHECK(ids.size() == B);
        for (std::uint32_t r = 0; r < B; ++r) {
            // Engine::sample_from on request b[r]
            SampleRequest& q = b[r];
            std::vector<float> row(host.begin() + (std::ptrdiff_t)r * STRIDE, host.begin() + (std::ptrdiff_t)r * STRIDE + V);
            const std::vector<float> raw = row;
            const TokenId next = sample(row, q.sampling, q.generated, q.rng, q.constraint);
            if (q.constraint) q.constraint->commit(next);
            q.generated.push_back(next);
            if (next != ids[r]) std::fprintf(stderr, "batch step %u row %u: batch %d per-row %d\n", step, r, ids[r], next);
            CHECK(next == ids[r]);
            CHECK(a[r].generated == q.generated);
            if (q.logprobs_opt.enabled) {
                float lp = 0.0f;
                std::vector<TokenLogprob> top;
                logprobs_from(raw, next, q.logprobs_opt.top, lp, top);
                const auto& e = a[r].logprobs.back();
                CHECK(e.token == next && std::fabs(e.logprob - lp) <= 1e-5f);
                CHECK(e.top.size() == top.size());
                for (std::size_t j = 0; j < top.size() && j < e.top.size(); ++j)
                    CHECK(e.top[j].token == top[j].token && std::fabs(e.top[j].logprob - top[j].logprob) <= 1e-5f);
            }
            // Engine::sample_from on request c[r], through the oracle
            SampleRequest& o = c[r];
            std::vector<float> orow(raw);
            OracleParams op;
            std::memcpy(&op, &o.sampling, sizeof op);
            const std::size_t nh = o.generated.size(), w = std::min<std::size_t>(nh, o.sampling.repeat_last_n);
            const double u = o.sampling.temperature > 0.0f ? std::generate_canonical<double, 53>(o.rng) : 0.0;
            const std::uint32_t* m = nullptr;
            if (o.constraint) {
                CHECK(o.constraint->allow_mask(V, words.data()));
                m = words.data();
            }
            const TokenId oid = orc.sample(orow.data(), V, &op, o.generated.data() + (nh - w),
                                           static_cast<std::uint32_t>(w), u, m, nullptr);
            if (o.constraint) o.constraint->commit(oid);
            o.generated.push_back(oid);
            if (oid != ids[r]) std::fprintf(stderr, "batch step %u row %u: batch %d oracle %d\n", step, r, ids[r], oid);
            CHECK(oid == ids[r]);
            CHECK(a[r].generated == o.generated);
            if (o.logprobs_opt.enabled) {
                const std::uint32_t k = std::min(o.logprobs_opt.top, V);
                float lp = 0.0f;
                std::vector<std::int32_t> tid(k + 1);
                std::vector<float> tlp(k + 1);
                orc.logprobs(raw.data(), V, oid, k, &lp, tid.data(), tlp.data(), nullptr);
                const auto& e = a[r].logprobs.back();
                CHECK(std::fabs(e.logprob - lp) <= 1e-5f);
                CHECK(e.top.size() == k);
                for (std::size_t j = 0; j < k && j < e.top.size(); ++j)
                    CHECK(e.top[j].token == tid[j] && std::fabs(e.top[j].logprob - tlp[j]) <= 1e-5f);
            }
        }
        // engine states compared without advancing them: one output per
        // stochastic row and step, none for greedy rows
        for (std::uint32_t r = 0; r < B; ++r) CHECK(a[r].rng == b[r].rng && a[r].rng == c[r].rng);
    }
    for (std::uint32_t t = 0; t < V; t += 97) {
        CHECK(ca.allows(static_cast<TokenId>(t)) == cb.allows(static_cast<TokenId>(t)));
        CHECK(ca.allows(static_cast<TokenId>(t)) == cc.allows(static_cast<TokenId>(t)));
    }
    (void)hipFree(dlog);
    // limits
    std::vector<SampleRequest> many(B + 1);
    std::vector<SampleRequest*> mp;
    for (auto& q : many) mp.push_back(&q);
    CHECK(throws<std::invalid_argument>([&] { bs.sample_step(nullptr, LCS_F32, STRIDE, mp); }));
    // a limit met by a later row rejects the step before any rng advances
    std::vector<SampleRequest> lim(2);
    lim[0].sampling.temperature = 1.0f;
    lim[0].rng.seed(7);
    lim[1].logprobs_opt = {true, 21};   // above max_top
    std::vector<SampleRequest*> lp{&lim[0], &lim[1]};
    CHECK(throws<std::invalid_argument>([&] { bs.sample_step(nullptr, LCS_F32, STRIDE, lp); }));
    std::mt19937_64 fresh(7);
    CHECK(lim[0].rng() == fresh());
    CHECK(lim[0].generated.empty() && lim[1].generated.empty());
}

// BatchSampler on steps whose rows are all min-p window rows: the penalty
// windows live in device slots that each step advances by the sampled id.
// Requests leave and rejoin (their slots are released and reloaded), one
// request's history is replaced between steps (the slot must reload), and
// one has penalties off. Every step's ids and logprobs are checked against
// the CPU oracle run on the request's whole history (sample_from,
// engine.cpp:423-450).
static void test_batch_gpu_windows() {
    using locus::engine::BatchSampler;
    using locus::sampler::SampleRequest;
    constexpr std::uint32_t V = 32003, B = 12, K = 8, STRIDE = (V + 3) / 4 * 4;
    const Oracle orc = load_oracle();
    std::mt19937_64 pr(23);
    std::vector<SampleRequest> a(B), c(B);
    for (std::uint32_t r = 0; r < B; ++r) {
        SamplingParams& p = a[r].sampling;
        p.temperature = 0.7f + 0.05f * (float)(r % 3);
        p.min_p = 0.05f;
        p.top_p = 0.9f;
        p.repeat_penalty = 1.1f;
        p.frequency_penalty = 0.5f;
        p.presence_penalty = 0.3f;
        p.repeat_last_n = r % 3 == 0 ? 64 : 2048;
        if (r == 5) p.repeat_penalty = 1.0f, p.frequency_penalty = 0.0f, p.presence_penalty = 0.0f;
        a[r].rng.seed(500 + r);
        const std::uint32_t n = r % 4 == 0 ? 3 : 200 + 100 * r;
        // few distinct ids, so that counts repeat and entries leave the window
        for (std::uint32_t i = 0; i < n; ++i) a[r].generated.push_back(static_cast<TokenId>(pr() % 700));
        a[r].logprobs_opt = {r % 2 == 0, 5u};
        c[r] = a[r];
    }
    BatchSampler bs(0, B, V, 4096, 20);
    float* dlog = nullptr;
    CHECK(hipMalloc(&dlog, (std::size_t)B * STRIDE * sizeof(float)) == hipSuccess);
    std::mt19937 lr(7);
    std::normal_distribution<float> nd(0.0f, 3.0f);
    std::vector<float> host((std::size_t)B * STRIDE, 0.0f);
    for (std::uint32_t step = 0; step < K; ++step) {
        // rows 0-3 sit out steps 3 and 4; row 7's history is replaced before step 5
        std::vector<std::uint32_t> in;
        for (std::uint32_t r = 0; r < B; ++r)
            if (!(r < 4 && (step == 3 || step == 4))) in.push_back(r);
        if (step == 5) {
            for (SampleRequest* q : {&a[7], &c[7]}) {
                q->generated.assign(150, 0);
                for (std::uint32_t i = 0; i < 150; ++i) q->generated[i] = static_cast<TokenId>((i * 37u) % 500u);
            }
        }
        std::vector<SampleRequest*> ap;
        for (std::uint32_t r : in) ap.push_back(&a[r]);
        const std::uint32_t n = static_cast<std::uint32_t>(in.size());
        for (std::uint32_t i = 0; i < n; ++i)
            for (std::uint32_t t = 0; t < V; ++t) host[(std::size_t)i * STRIDE + t] = nd(lr);
        CHECK(hipMemcpy(dlog, host.data(), (std::size_t)n * STRIDE * sizeof(float), hipMemcpyHostToDevice) ==
              hipSuccess);
        const std::vector<TokenId> ids = bs.sample_step(dlog, LCS_F32, STRIDE, ap);
        CHECK(ids.size() == n);
        for (std::uint32_t i = 0; i < n; ++i) {
            SampleRequest& o = c[in[i]];
            std::vector<float> raw(host.begin() + (std::ptrdiff_t)i * STRIDE,
                                   host.begin() + (std::ptrdiff_t)i * STRIDE + V);
            std::vector<float> row(raw);
            OracleParams op;
            std::memcpy(&op, &o.sampling, sizeof op);
            const std::size_t nh = o.generated.size(), w = std::min<std::size_t>(nh, o.sampling.repeat_last_n);
            const double u = std::generate_canonical<double, 53>(o.rng);
            const TokenId oid = orc.sample(row.data(), V, &op, o.generated.data() + (nh - w),
                                           static_cast<std::uint32_t>(w), u, nullptr, nullptr);
            o.generated.push_back(oid);
            if (oid != ids[i]) std::fprintf(stderr, "window step %u row %u: batch %d oracle %d\n", step, in[i], ids[i], oid);
            CHECK(oid == ids[i]);
            CHECK(a[in[i]].generated == o.generated);
            if (o.logprobs_opt.enabled) {
                float lp = 0.0f;
                std::vector<std::int32_t> tid(6);
                std::vector<float> tlp(6);
                orc.logprobs(raw.data(), V, oid, 5, &lp, tid.data(), tlp.data(), nullptr);
                const auto& e = a[in[i]].logprobs.back();
                CHECK(std::fabs(e.logprob - lp) <= 1e-5f);
                CHECK(e.top.size() == 5);
                for (std::size_t j = 0; j < 5 && j < e.top.size(); ++j)
                    CHECK(e.top[j].token == tid[j] && std::fabs(e.top[j].logprob - tlp[j]) <= 1e-5f);
            }
        }
        for (std::uint32_t r : in) CHECK(a[r].rng == c[r].rng);
    }
    (void)hipFree(dlog);
}

// A row the device could not serve (id -1, locus_sampler.h) fails the step;
// the status word is read only then.
static void test_unserved_rows() {
    int reads = 0;
    auto status = [&] { ++reads; return 2u; };
    const std::int32_t ok[3] = {5, 0, 7};
    locus::engine::detail::check_served(ok, 3, status);
    CHECK(reads == 0);
    const std::int32_t bad[3] = {5, -1, 7};
    bool thrown = false;
    try {
        locus::engine::detail::check_served(bad, 3, status);
    } catch (const std::runtime_error& e) {
        thrown = std::string(e.what()).find("row 1") != std::string::npos &&
                 std::string(e.what()).find("status 2") != std::string::npos;
    }
    CHECK(thrown);
    CHECK(reads == 1);
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        if (mode == "cpu") {
            test_grammar();
            test_mask_builder();
            test_ngram();
            test_registry(false);
            test_unserved_rows();
        } else if (mode == "gpu") {
            test_registry(true);
            test_sampling_gpu();
            test_batch_gpu();
            test_batch_gpu_windows();
        } else {
            std::fprintf(stderr, "usage: test_host cpu|gpu\n");
            return 2;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d checks passed, %d failed\n", mode.c_str(), g_pass, g_fail);
    return g_fail == 0 ? 0 : 1;
}
