// CPU ORACLE — TEST INFRASTRUCTURE ONLY.
//
// A plain C++ restatement of the reference sampler path, used exclusively by
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
// checker. Nothing in the product (locus_amd/, include/) links, loads or calls
// this file. Built with g++ -O2 -ffp-contract=off so that no FMA contraction
// changes a rounding (the reference's x86-64 build never contracts
// sampling.cpp: CMakeLists.txt:83-99 gives -mfma only to matvec_avx2.cpp).
//
// Functions and the reference lines they restate:
//   orc_sample        src/locus/model/sampling.cpp:45-148 (sample) with
//                     apply_penalties sampling.cpp:16-41 and, for the greedy
//                     branch, argmax src/locus/model/llama.cpp:1237-1245.
//                     The draw is std::uniform_real_distribution<double>
//                     (0, kept_sum) over one mt19937_64 output, i.e.
//                     r = u * (kept_sum - 0) + 0 with u from
//                     generate_canonical (libstdc++ random.tcc:3348-3380,
//                     random.h:1868-1870); u is passed in.
//   orc_logprobs      sampling.cpp:150-190 (logprobs_from).
//   orc_argmax        llama.cpp:1237-1245.
//   orc_json_*        src/locus/model/grammar.cpp:16-201 (JsonGrammar) and the
//                     per-token allows() of server.cpp:154-185.
//   orc_ngram_draft   src/locus/model/speculative.cpp:7-28.
//   orc_verify        engine.cpp:357-396 acceptance rule + logprobs_from
//                     (chosen = draft, n_top = 0) per row.
//   orc_mt_u          generate_canonical<double,53>(std::mt19937_64(seed))
//                     after `skip` discarded outputs.
//
// Beyond the reference's outputs the oracle reports diagnostics that the
// reference computes but does not return (survivor counts, boundary logit,
// normaliser) plus decision margins: the distance of each decisive comparison
// from its threshold, in CDF units. Tests use the margins to identify the
// documented near-tie rows and the tie flags for exact-tie rows.
//
// Parity pinning (what checks each function, all in tests/test_oracle.py):
//   orc_sample/orc_logprobs/orc_argmax: golden vectors produced by the
//     compiled reference (oracle/_ref) in tests/golden/configs.json and
//     edge.json, the reference's own KATs (tests/test_sampling.cpp), and
//     closed forms (numpy log-softmax, brute-force sorted prefixes).
//   orc_json_feed/orc_json_complete: the compiled reference's accept counts
//     and complete() on 353 golden strings (tests/golden/grammar.json) and the
//     reference's KATs (tests/test_grammar.cpp:28-77).
//   orc_json_mask: the compiled reference's masks in grammar.json.
//   orc_ngram_draft: the compiled reference's drafts on 200 golden cases
//     (tests/golden/ngram.json), its KATs (tests/test_speculative.cpp:9-32)
//     and a brute-force statement of the rule.
//   orc_verify: golden argmax / draft logprob / acceptance in configs.json.
//   orc_mt_u: the C++ standard's check value for mt19937_64 ([rand.predef]).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

extern "C" {

typedef struct orc_params {
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float repeat_penalty;
    float frequency_penalty;
    float presence_penalty;
    uint32_t repeat_last_n;
} orc_params;

typedef struct orc_diag {
    int32_t id;
    uint32_t n_cand;     // candidates after the constraint (all if none allowed)
    uint32_t keep_topk;  // candidate count after top-k
    uint32_t keep_p;     // prefix length after top-p
    uint32_t keep;       // final survivor count (after min-p)
    uint32_t pos;        // sorted position of the drawn token
    float maxl;          // cand[0] logit (max after penalties/mask/top-k)
    float boundary;      // cand[keep-1] logit
    double sum;          // softmax normaliser over the candidate list
    double kept_sum;
    double r;            // u * kept_sum
    double margin_p;     // min |cum_i - top_p| over the decisive i
    double margin_m;     // min |w_i/sum - thresh| / thresh over the decisive i
    double margin_r;     // min |r_i| / kept_sum over the decisive i
    uint32_t tie_flags;  // 1 top-k cut, 2 keep boundary, 4 drawn position
    uint32_t greedy;     // 1 when the greedy branch ran
} orc_diag;

}  // extern "C"

namespace {

constexpr double kInf = std::numeric_limits<double>::infinity();

bool mask_allows(const uint32_t* mask, uint32_t t) {
    return (mask[t >> 5] >> (t & 31u)) & 1u;
}

void penalties(float* logits, uint32_t V, const orc_params& p,
               const int32_t* hist, uint32_t n_hist) {
    if (p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f &&
        p.presence_penalty == 0.0f) {
        return;
    }
    const std::size_t n = n_hist;
    const std::size_t first = n > p.repeat_last_n ? n - p.repeat_last_n : 0;
    std::unordered_map<int32_t, int> count;
    for (std::size_t i = first; i < n; ++i) {
        ++count[hist[i]];
    }
    for (const auto& kv : count) {
        if (static_cast<std::size_t>(kv.first) >= V) {
            continue;  // ids >= V and negative ids (size_t wrap) are skipped
        }
        float& l = logits[kv.first];
        if (p.repeat_penalty != 1.0f) {
            l = l > 0.0f ? l / p.repeat_penalty : l * p.repeat_penalty;
        }
        l -= p.frequency_penalty * static_cast<float>(kv.second) +
             p.presence_penalty;
    }
}

int32_t argmax_span(const float* l, uint32_t V) {
    std::size_t best = 0;
    for (std::size_t i = 1; i < V; ++i) {
        if (l[i] > l[best]) {
            best = i;
        }
    }
    return static_cast<int32_t>(best);
}

int32_t sample_impl(float* logits, uint32_t V, const orc_params& p,
                    const int32_t* hist, uint32_t n_hist, double u,
                    const uint32_t* mask, orc_diag* d) {
    orc_diag dd{};
    dd.margin_p = dd.margin_m = dd.margin_r = kInf;
    penalties(logits, V, p, hist, n_hist);

    if (p.temperature <= 0.0f) {
        dd.greedy = 1;
        int32_t id;
        if (mask == nullptr) {
            id = argmax_span(logits, V);
        } else {
            int64_t best = -1;
            float best_l = 0.0f;
            for (uint32_t i = 0; i < V; ++i) {
                if (mask_allows(mask, i) && (best < 0 || logits[i] > best_l)) {
                    best = i;
                    best_l = logits[i];
                }
            }
            id = best >= 0 ? static_cast<int32_t>(best) : argmax_span(logits, V);
        }
        dd.id = id;
        if (d) *d = dd;
        return id;
    }

    std::vector<std::pair<float, uint32_t>> cand;
    cand.reserve(V);
    for (uint32_t i = 0; i < V; ++i) {
        cand.emplace_back(logits[i], i);
    }
    if (mask != nullptr) {
        std::vector<std::pair<float, uint32_t>> allowed;
        allowed.reserve(cand.size());
        for (const auto& c : cand) {
            if (mask_allows(mask, c.second)) {
                allowed.push_back(c);
            }
        }
        if (!allowed.empty()) {
            cand.swap(allowed);
        }
    }
    dd.n_cand = static_cast<uint32_t>(cand.size());
    const auto desc = [](const std::pair<float, uint32_t>& a,
                         const std::pair<float, uint32_t>& b) {
        return a.first > b.first;
    };
    if (p.top_k > 0 && p.top_k < static_cast<uint32_t>(cand.size())) {
        std::partial_sort(cand.begin(), cand.begin() + p.top_k, cand.end(), desc);
        // diagnostic: does an unselected candidate tie the k-th?
        const float kth = cand[p.top_k - 1].first;
        for (std::size_t i = p.top_k; i < cand.size(); ++i) {
            if (cand[i].first == kth) {
                dd.tie_flags |= 1u;
                break;
            }
        }
        cand.resize(p.top_k);
    } else {
        std::sort(cand.begin(), cand.end(), desc);
    }
    dd.keep_topk = static_cast<uint32_t>(cand.size());

    const float maxl = cand.front().first;
    const float inv_t = 1.0f / p.temperature;
    double sum = 0.0;
    std::vector<double> w(cand.size());
    for (std::size_t i = 0; i < cand.size(); ++i) {
        w[i] = std::exp(static_cast<double>((cand[i].first - maxl) * inv_t));
        sum += w[i];
    }

    std::size_t keep = cand.size();
    if (p.top_p < 1.0f) {
        double cum = 0.0;
        double prev = -kInf;
        bool hit = false;
        for (std::size_t i = 0; i < cand.size(); ++i) {
            cum += w[i] / sum;
            if (cum >= p.top_p) {
                keep = i + 1;
                dd.margin_p = cum - static_cast<double>(p.top_p);
                if (i > 0) {
                    dd.margin_p = std::min(dd.margin_p,
                                           static_cast<double>(p.top_p) - prev);
                }
                hit = true;
                break;
            }
            prev = cum;
        }
        if (!hit) {
            dd.margin_p = static_cast<double>(p.top_p) - prev;
        }
    }
    dd.keep_p = static_cast<uint32_t>(keep);
    if (p.min_p > 0.0f) {
        const double thresh = p.min_p * (w[0] / sum);
        bool cut = false;
        double last_ok = kInf;
        for (std::size_t i = 1; i < keep; ++i) {
            const double q = w[i] / sum;
            if (q < thresh) {
                dd.margin_m = std::min((thresh - q) / thresh,
                                       (last_ok - thresh) / thresh);
                keep = i;
                cut = true;
                break;
            }
            last_ok = q;
        }
        if (!cut && keep >= 2) {
            dd.margin_m = (last_ok - thresh) / thresh;
        }
    }
    dd.keep = static_cast<uint32_t>(keep);
    if (keep < cand.size() && cand[keep].first == cand[keep - 1].first) {
        dd.tie_flags |= 2u;
    }

    double kept_sum = 0.0;
    for (std::size_t i = 0; i < keep; ++i) {
        kept_sum += w[i];
    }
    double r = u * (kept_sum - 0.0) + 0.0;
    dd.r = r;
    std::size_t chosen = keep - 1;
    double before = r;
    bool found = false;
    for (std::size_t i = 0; i < keep; ++i) {
        r -= w[i];
        if (r <= 0.0) {
            chosen = i;
            dd.margin_r = std::min(-r, before) / kept_sum;
            found = true;
            break;
        }
        before = r;
    }
    if (!found) {
        dd.margin_r = std::fabs(r) / kept_sum;
    }
    if ((chosen + 1 < cand.size() && cand[chosen + 1].first == cand[chosen].first) ||
        (chosen > 0 && cand[chosen - 1].first == cand[chosen].first)) {
        dd.tie_flags |= 4u;
    }
    dd.id = static_cast<int32_t>(cand[chosen].second);
    dd.pos = static_cast<uint32_t>(chosen);
    dd.maxl = maxl;
    dd.boundary = cand[keep - 1].first;
    dd.sum = sum;
    dd.kept_sum = kept_sum;
    if (d) *d = dd;
    return dd.id;
}

void logprobs_impl(const float* logits, uint32_t V, int32_t chosen,
                   uint32_t n_top, float* chosen_lp, int32_t* top_ids,
                   float* top_lp, uint32_t* tie) {
    float max_logit = logits[0];
    for (uint32_t i = 0; i < V; ++i) {
        max_logit = std::max(max_logit, logits[i]);
    }
    double s = 0.0;
    for (uint32_t i = 0; i < V; ++i) {
        s += std::exp(static_cast<double>(logits[i]) - max_logit);
    }
    const double log_z = std::log(s) + max_logit;
    const auto lp = [&](std::size_t i) {
        return static_cast<float>(logits[i] - log_z);
    };
    *chosen_lp = (chosen >= 0 && static_cast<uint32_t>(chosen) < V)
                     ? lp(static_cast<std::size_t>(chosen))
                     : 0.0f;
    if (tie) *tie = 0;
    const std::size_t k = std::min<std::size_t>(n_top, V);
    if (k == 0) {
        return;
    }
    std::vector<std::size_t> idx(V);
    for (std::size_t i = 0; i < V; ++i) idx[i] = i;
    std::partial_sort(idx.begin(), idx.begin() + k, idx.end(),
                      [&](std::size_t a, std::size_t b) {
                          return logits[a] > logits[b];
                      });
    for (std::size_t i = 0; i < k; ++i) {
        top_ids[i] = static_cast<int32_t>(idx[i]);
        top_lp[i] = lp(idx[i]);
    }
    if (tie) {
        // tie flag: some element outside the top-k equals the k-th value, or
        // equal values inside the top-k (their order is unspecified).
        const float kth = logits[idx[k - 1]];
        for (std::size_t i = k; i < V; ++i) {
            if (logits[idx[i]] == kth) { *tie = 1; break; }
        }
        for (std::size_t i = 1; i < k; ++i) {
            if (logits[idx[i]] == logits[idx[i - 1]]) { *tie = 1; break; }
        }
    }
}

// ----- JsonGrammar restatement (grammar.cpp:16-201) -----
enum class GS : uint8_t {
    Val, ArrStart, ObjStart, ObjKey, Colon, InStr, StrEsc, StrU, InNum, Kw, AfterVal
};

struct Json {
    std::vector<char> stack;
    GS st = GS::Val;
    bool in_key = false;
    bool num_digit = false;
    int u_left = 0;
    std::string kw;

    static bool ws(uint8_t b) { return b == ' ' || b == '\t' || b == '\n' || b == '\r'; }
    static bool dig(uint8_t b) { return b >= '0' && b <= '9'; }
    static bool hex(uint8_t b) {
        return dig(b) || (b >= 'a' && b <= 'f') || (b >= 'A' && b <= 'F');
    }
    bool begin(uint8_t b) {
        switch (b) {
            case '{': stack.push_back('{'); st = GS::ObjStart; return true;
            case '[': stack.push_back('['); st = GS::ArrStart; return true;
            case '"': st = GS::InStr; in_key = false; return true;
            case 't': st = GS::Kw; kw = "rue"; return true;
            case 'f': st = GS::Kw; kw = "alse"; return true;
            case 'n': st = GS::Kw; kw = "ull"; return true;
            default: break;
        }
        if (b == '-' || dig(b)) {
            st = GS::InNum;
            num_digit = dig(b);
            return true;
        }
        return false;
    }
    bool feed(uint8_t b) {
        for (;;) {
            switch (st) {
                case GS::Val:
                case GS::ArrStart:
                    if (ws(b)) return true;
                    if (st == GS::ArrStart && b == ']') {
                        stack.pop_back();
                        st = GS::AfterVal;
                        return true;
                    }
                    return begin(b);
                case GS::ObjStart:
                    if (ws(b)) return true;
                    if (b == '}') { stack.pop_back(); st = GS::AfterVal; return true; }
                    if (b == '"') { st = GS::InStr; in_key = true; return true; }
                    return false;
                case GS::ObjKey:
                    if (ws(b)) return true;
                    if (b == '"') { st = GS::InStr; in_key = true; return true; }
                    return false;
                case GS::Colon:
                    if (ws(b)) return true;
                    if (b == ':') { st = GS::Val; return true; }
                    return false;
                case GS::InStr:
                    if (b == '"') {
                        if (in_key) { in_key = false; st = GS::Colon; }
                        else { st = GS::AfterVal; }
                        return true;
                    }
                    if (b == '\\') { st = GS::StrEsc; return true; }
                    return b >= 0x20;
                case GS::StrEsc:
                    if (b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' ||
                        b == 'n' || b == 'r' || b == 't') {
                        st = GS::InStr;
                        return true;
                    }
                    if (b == 'u') { st = GS::StrU; u_left = 4; return true; }
                    return false;
                case GS::StrU:
                    if (hex(b)) {
                        if (--u_left == 0) st = GS::InStr;
                        return true;
                    }
                    return false;
                case GS::InNum:
                    if (dig(b)) { num_digit = true; return true; }
                    if (b == '.' || b == 'e' || b == 'E' || b == '+' || b == '-') return true;
                    if (!num_digit) return false;
                    st = GS::AfterVal;
                    continue;
                case GS::Kw:
                    if (!kw.empty() && b == static_cast<uint8_t>(kw.front())) {
                        kw.erase(kw.begin());
                        if (kw.empty()) st = GS::AfterVal;
                        return true;
                    }
                    return false;
                case GS::AfterVal:
                    if (ws(b)) return true;
                    if (stack.empty()) return false;
                    if (stack.back() == '[') {
                        if (b == ',') { st = GS::Val; return true; }
                        if (b == ']') { stack.pop_back(); st = GS::AfterVal; return true; }
                        return false;
                    }
                    if (b == ',') { st = GS::ObjKey; return true; }
                    if (b == '}') { stack.pop_back(); st = GS::AfterVal; return true; }
                    return false;
            }
        }
    }
    bool complete() const {
        return stack.empty() && (st == GS::AfterVal || (st == GS::InNum && num_digit));
    }
};

}  // namespace

extern "C" {

int32_t orc_sample(float* logits, uint32_t V, const orc_params* p,
                   const int32_t* hist, uint32_t n_hist, double u,
                   const uint32_t* mask, orc_diag* diag) {
    return sample_impl(logits, V, *p, hist, n_hist, u, mask, diag);
}

void orc_logprobs(const float* logits, uint32_t V, int32_t chosen,
                  uint32_t n_top, float* chosen_lp, int32_t* top_ids,
                  float* top_lp, uint32_t* tie) {
    logprobs_impl(logits, V, chosen, n_top, chosen_lp, top_ids, top_lp, tie);
}

int32_t orc_argmax(const float* logits, uint32_t V) { return argmax_span(logits, V); }

// Batched engine-style driver (engine.cpp:423-450 per row, rows in order):
// raw snapshot when logprobs are on, sample (mutating the row in place),
// logprobs on the snapshot. `threads` > 1 spreads rows over std::threads.
// mask may be NULL; has_mask (per row) may be NULL meaning every row masked.
void orc_sample_batch(float* logits, uint32_t rows, uint32_t V, uint64_t row_stride,
                      const orc_params* params, const uint32_t* hist_off,
                      const int32_t* hist_ids, const double* u,
                      const uint32_t* mask, const uint8_t* has_mask,
                      uint32_t mask_words, int want_logprobs, uint32_t n_top,
                      int32_t* ids, float* chosen_lp, int32_t* top_ids,
                      float* top_lp, orc_diag* diag, uint32_t threads) {
    auto run = [&](uint32_t r0, uint32_t r1) {
        std::vector<float> raw;
        for (uint32_t r = r0; r < r1; ++r) {
            float* row = logits + static_cast<uint64_t>(r) * row_stride;
            if (want_logprobs) raw.assign(row, row + V);
            const int32_t* h = hist_off ? hist_ids + hist_off[r] : nullptr;
            const uint32_t nh = hist_off ? hist_off[r + 1] - hist_off[r] : 0;
            const uint32_t* m = nullptr;
            if (mask && (has_mask == nullptr || has_mask[r])) {
                m = mask + static_cast<uint64_t>(r) * mask_words;
            }
            ids[r] = sample_impl(row, V, params[r], h, nh, u ? u[r] : 0.0, m,
                                 diag ? diag + r : nullptr);
            if (want_logprobs) {
                logprobs_impl(raw.data(), V, ids[r], n_top, chosen_lp + r,
                              top_ids + static_cast<uint64_t>(r) * n_top,
                              top_lp + static_cast<uint64_t>(r) * n_top, nullptr);
            }
        }
    };
    if (threads <= 1) {
        run(0, rows);
        return;
    }
    std::vector<std::thread> pool;
    const uint32_t per = (rows + threads - 1) / threads;
    for (uint32_t t = 0; t < threads; ++t) {
        const uint32_t r0 = t * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) pool.emplace_back(run, r0, r1);
    }
    for (auto& th : pool) th.join();
}

// Speculative verify per row (engine.cpp:357-396 with logprobs_from
// sampling.cpp:150-190): argmax, lp(draft), acceptance per sequence.
void orc_verify(const void* logits, int bf16, uint32_t n_seq, uint32_t rows_per_seq,
                uint32_t V, uint64_t row_stride, const int32_t* draft,
                int32_t* argmax_ids, float* draft_lp, uint32_t* accept_len,
                uint32_t threads) {
    const uint32_t rows = n_seq * rows_per_seq;
    auto run = [&](uint32_t r0, uint32_t r1) {
        std::vector<float> row(V);
        for (uint32_t r = r0; r < r1; ++r) {
            if (bf16) {
                const uint16_t* src = static_cast<const uint16_t*>(logits) + r * row_stride;
                for (uint32_t i = 0; i < V; ++i) {
                    const uint32_t bits = static_cast<uint32_t>(src[i]) << 16;
                    std::memcpy(&row[i], &bits, 4);
                }
            } else {
                const float* src = static_cast<const float*>(logits) + r * row_stride;
                std::memcpy(row.data(), src, V * sizeof(float));
            }
            argmax_ids[r] = argmax_span(row.data(), V);
            logprobs_impl(row.data(), V, draft[r], 0, draft_lp + r, nullptr, nullptr, nullptr);
        }
    };
    if (threads <= 1) {
        run(0, rows);
    } else {
        std::vector<std::thread> pool;
        const uint32_t per = (rows + threads - 1) / threads;
        for (uint32_t t = 0; t < threads; ++t) {
            const uint32_t r0 = t * per, r1 = std::min(rows, r0 + per);
            if (r0 < r1) pool.emplace_back(run, r0, r1);
        }
        for (auto& th : pool) th.join();
    }
    for (uint32_t s = 0; s < n_seq; ++s) {
        uint32_t acc = 0;
        while (acc < rows_per_seq &&
               argmax_ids[s * rows_per_seq + acc] == draft[s * rows_per_seq + acc]) {
            ++acc;
        }
        accept_len[s] = acc;
    }
}

// mt19937_64(seed), discard `skip` outputs, then one generate_canonical.
double orc_mt_u(uint64_t seed, uint64_t skip) {
    std::mt19937_64 g(seed);
    g.discard(skip);
    return std::generate_canonical<double, 53>(g);
}
uint64_t orc_mt_raw(uint64_t seed, uint64_t skip) {
    std::mt19937_64 g(seed);
    g.discard(skip);
    return g();
}

// JsonGrammar handle API.
void* orc_json_new(void) { return new Json(); }
void* orc_json_clone(const void* g) { return new Json(*static_cast<const Json*>(g)); }
void orc_json_free(void* g) { delete static_cast<Json*>(g); }
int orc_json_feed(void* g, uint8_t b) { return static_cast<Json*>(g)->feed(b) ? 1 : 0; }
int orc_json_complete(const void* g) { return static_cast<const Json*>(g)->complete() ? 1 : 0; }

// Brute-force allow-mask: bit t set iff feeding piece t into a copy of `g`
// accepts every byte (server.cpp:160-171); ids >= n_pieces are allowed.
void orc_json_mask(const void* g, const uint8_t* blob, const uint64_t* off,
                   uint32_t n_pieces, uint32_t V, uint32_t* mask_out) {
    const Json& live = *static_cast<const Json*>(g);
    const uint32_t words = (V + 31) / 32;
    std::memset(mask_out, 0, words * sizeof(uint32_t));
    for (uint32_t t = 0; t < V; ++t) {
        bool ok = true;
        if (t < n_pieces) {
            Json c = live;
            for (uint64_t b = off[t]; b < off[t + 1]; ++b) {
                if (!c.feed(blob[b])) { ok = false; break; }
            }
        }
        if (ok) mask_out[t >> 5] |= 1u << (t & 31u);
    }
}

// Prompt-lookup draft (speculative.cpp:7-28). Returns the draft length.
uint32_t orc_ngram_draft(const int32_t* ctx, uint32_t n, uint32_t ngram,
                         uint32_t max_draft, int32_t* out) {
    if (ngram == 0 || max_draft == 0 || n <= ngram) return 0;
    const int32_t* pat = ctx + (n - ngram);
    for (std::size_t start = n - ngram; start-- > 0;) {
        if (std::equal(pat, pat + ngram, ctx + start)) {
            uint32_t k = 0;
            for (std::size_t i = start + ngram; i < n && k < max_draft; ++i) {
                out[k++] = ctx[i];
            }
            return k;
        }
    }
    return 0;
}

uint32_t orc_sizeof_diag(void) { return sizeof(orc_diag); }

}  // extern "C"
