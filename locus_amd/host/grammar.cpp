// Host JSON grammar, trie mask builder and JSON token constraint
// (reference: src/locus/model/grammar.cpp, src/locus/server/server.cpp:154-185).
#include "locus/model/grammar.hpp"

#include <algorithm>
#include <cstring>
#include <numeric>

namespace locus::model {

namespace {

constexpr const char* kKeywords[3] = {"true", "false", "null"};
constexpr std::uint8_t kKeywordLen[3] = {4, 5, 4};

bool space(std::uint8_t b) { return b == ' ' || b == '\t' || b == '\n' || b == '\r'; }
bool digit(std::uint8_t b) { return b >= '0' && b <= '9'; }
bool hex(std::uint8_t b) {
    return digit(b) || (b >= 'a' && b <= 'f') || (b >= 'A' && b <= 'F');
}
// bytes allowed after a backslash other than 'u' (grammar.cpp:120-131)
bool simple_escape(std::uint8_t b) {
    return std::strchr("\"\\/bfnrt", b) != nullptr && b != 0;
}

}  // namespace

// value start (grammar.cpp:16-53): containers push, scalars enter their mode
bool JsonGrammar::start_value(std::uint8_t b) {
    switch (b) {
        case '{': open_.push_back('{'); mode_ = kObjectOpen; return true;
        case '[': open_.push_back('['); mode_ = kArrayOpen; return true;
        case '"': mode_ = kString; bits_ &= ~kInKey; return true;
        case 't': mode_ = kKeyword; aux_ = (0u << 4) | 1u; return true;
        case 'f': mode_ = kKeyword; aux_ = (1u << 4) | 1u; return true;
        case 'n': mode_ = kKeyword; aux_ = (2u << 4) | 1u; return true;
        default: break;
    }
    if (b == '-' || digit(b)) {
        mode_ = kNumber;
        bits_ = digit(b) ? (bits_ | kNumDigit) : (bits_ & ~kNumDigit);
        return true;
    }
    return false;
}

// closes the innermost container if it is `want`
bool JsonGrammar::close(char want) {
    if (open_.empty() || open_.back() != want) return false;
    open_.pop_back();
    mode_ = kDone;
    return true;
}

bool JsonGrammar::feed(std::uint8_t b) {
    switch (mode_) {
        case kValue:
            return space(b) || start_value(b);
        case kArrayOpen:
            if (space(b)) return true;
            return b == ']' ? close('[') : start_value(b);
        case kObjectOpen:
        case kKey:
            if (space(b)) return true;
            if (mode_ == kObjectOpen && b == '}') return close('{');
            if (b != '"') return false;
            mode_ = kString;
            bits_ |= kInKey;
            return true;
        case kColon:
            if (space(b)) return true;
            if (b != ':') return false;
            mode_ = kValue;
            return true;
        case kString:
            if (b == '"') {
                mode_ = (bits_ & kInKey) ? kColon : kDone;
                bits_ &= ~kInKey;
                return true;
            }
            if (b == '\\') { mode_ = kEscape; return true; }
            return b >= 0x20;
        case kEscape:
            if (b == 'u') { mode_ = kUnicode; aux_ = 4; return true; }
            if (!simple_escape(b)) return false;
            mode_ = kString;
            return true;
        case kUnicode:
            if (!hex(b)) return false;
            if (--aux_ == 0) mode_ = kString;
            return true;
        case kNumber:
            if (digit(b)) { bits_ |= kNumDigit; return true; }
            if (b == '.' || b == 'e' || b == 'E' || b == '+' || b == '-') return true;
            if (!(bits_ & kNumDigit)) return false;
            mode_ = kDone;   // the number ends; b is read again as what follows it
            return feed(b);
        case kKeyword: {
            const std::uint8_t id = aux_ >> 4, got = aux_ & 15u;
            if (b != static_cast<std::uint8_t>(kKeywords[id][got])) return false;
            aux_ = static_cast<std::uint8_t>((id << 4) | (got + 1));
            if (got + 1 == kKeywordLen[id]) mode_ = kDone;
            return true;
        }
        case kDone:
            if (space(b)) return true;
            if (open_.empty()) return false;   // a finished top-level value takes only whitespace
            if (b == ',') {
                mode_ = open_.back() == '[' ? kValue : kKey;
                return true;
            }
            return b == (open_.back() == '[' ? ']' : '}') && close(open_.back());
    }
    return false;
}

bool JsonGrammar::complete() const {
    return open_.empty() && (mode_ == kDone || (mode_ == kNumber && (bits_ & kNumDigit)));
}

JsonGrammar::Mark JsonGrammar::mark() const {
    return Mark{mode_, bits_, aux_, open_.empty() ? std::uint8_t(0) : static_cast<std::uint8_t>(open_.back()),
                static_cast<std::uint32_t>(open_.size())};
}

void JsonGrammar::undo(const Mark& m) {
    if (open_.size() > m.depth) open_.pop_back();
    else if (open_.size() < m.depth) open_.push_back(static_cast<char>(m.top));
    mode_ = m.mode;
    bits_ = m.bits;
    aux_ = m.aux;
}

void JsonGrammar::state_key(std::uint32_t max_len, std::string& key) const {
    const std::uint32_t depth = static_cast<std::uint32_t>(open_.size());
    const std::uint32_t seen = std::min(depth, max_len);
    const std::uint32_t dk = std::min(depth, max_len + 1);
    key.push_back(static_cast<char>(mode_));
    key.push_back(static_cast<char>(bits_));
    key.push_back(static_cast<char>(aux_));
    key.append(reinterpret_cast<const char*>(&dk), sizeof dk);
    key.append(open_, depth - seen, seen);
}

JsonMaskBuilder::JsonMaskBuilder(std::vector<std::string> pieces, std::size_t cache_entries)
    : pieces_(std::move(pieces)), cache_cap_(cache_entries) {
    // build the trie from the pieces in lexicographic order: one pass, each
    // piece shares the prefix of the previous one
    std::vector<tok::TokenId> order(pieces_.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](tok::TokenId a, tok::TokenId b) {
        return pieces_[a] < pieces_[b];
    });
    nodes_.emplace_back();   // root
    std::vector<std::uint32_t> path{0};     // nodes along the previous piece
    std::vector<std::uint32_t> last_child{0};
    const std::string* prev = nullptr;
    toks_.reserve(order.size());
    for (tok::TokenId t : order) {
        const std::string& s = pieces_[t];
        max_len_ = std::max<std::uint32_t>(max_len_, static_cast<std::uint32_t>(s.size()));
        std::size_t common = 0;
        if (prev) {
            const std::size_t lim = std::min(prev->size(), s.size());
            while (common < lim && (*prev)[common] == s[common]) ++common;
        }
        path.resize(common + 1);
        last_child.resize(common + 1);
        for (std::size_t i = common; i < s.size(); ++i) {
            const std::uint32_t parent = path.back();
            const std::uint32_t id = static_cast<std::uint32_t>(nodes_.size());
            nodes_.emplace_back();
            nodes_[id].byte = static_cast<std::uint8_t>(s[i]);
            if (last_child.back() == 0) nodes_[parent].child = id;
            else nodes_[last_child.back()].sibling = id;
            last_child.back() = id;
            path.push_back(id);
            last_child.push_back(0);
        }
        Node& end = nodes_[path.back()];
        if (end.tok_end == 0 && end.tok_begin == 0) end.tok_begin = static_cast<std::uint32_t>(toks_.size());
        toks_.push_back(t);
        end.tok_end = static_cast<std::uint32_t>(toks_.size());
        prev = &s;
    }
}

void JsonMaskBuilder::walk(JsonGrammar g, std::uint32_t vocab, std::uint32_t* words) const {
    const std::uint32_t nw = (vocab + 31) / 32;
    std::fill(words, words + nw, 0u);
    auto allow = [&](tok::TokenId t) {
        if (static_cast<std::uint32_t>(t) < vocab) words[t >> 5] |= 1u << (t & 31);
    };
    for (std::uint32_t t = n_pieces(); t < vocab; ++t) allow(static_cast<tok::TokenId>(t));
    for (std::uint32_t i = nodes_[0].tok_begin; i < nodes_[0].tok_end; ++i) allow(toks_[i]);  // empty pieces
    // depth-first over the trie; a frame undoes its node's byte when it is left
    struct Frame {
        std::uint32_t next;
        JsonGrammar::Mark before;
    };
    std::vector<Frame> st;
    st.reserve(max_len_ + 2);
    st.push_back({nodes_[0].child, g.mark()});
    while (!st.empty()) {
        Frame& f = st.back();
        const std::uint32_t c = f.next;
        if (c == 0) {
            const JsonGrammar::Mark m = f.before;
            st.pop_back();
            g.undo(m);
            continue;
        }
        f.next = nodes_[c].sibling;
        const JsonGrammar::Mark m = g.mark();
        if (!g.feed(nodes_[c].byte)) {
            g.undo(m);
            continue;
        }
        for (std::uint32_t i = nodes_[c].tok_begin; i < nodes_[c].tok_end; ++i) allow(toks_[i]);
        st.push_back({nodes_[c].child, m});
    }
}

void JsonMaskBuilder::build(const JsonGrammar& g, std::uint32_t vocab, std::uint32_t* words) const {
    std::string key(reinterpret_cast<const char*>(&vocab), sizeof vocab);
    g.state_key(max_len_, key);
    const std::uint32_t nw = (vocab + 31) / 32;
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = index_.find(key);
        if (it != index_.end()) {
            lru_.splice(lru_.begin(), lru_, it->second);
            std::copy(it->second->second.begin(), it->second->second.end(), words);
            ++hits_;
            return;
        }
        ++misses_;
    }
    walk(g, vocab, words);
    if (cache_cap_ == 0) return;
    std::lock_guard<std::mutex> lk(mu_);
    if (index_.count(key)) return;
    lru_.emplace_front(key, std::vector<std::uint32_t>(words, words + nw));
    index_[key] = lru_.begin();
    if (lru_.size() > cache_cap_) {
        index_.erase(lru_.back().first);
        lru_.pop_back();
    }
}

std::pair<std::uint64_t, std::uint64_t> JsonMaskBuilder::cache_stats() const {
    std::lock_guard<std::mutex> lk(mu_);
    return {hits_, misses_};
}

bool JsonTokenConstraint::allows(tok::TokenId t) const {
    if (t < 0 || static_cast<std::uint32_t>(t) >= pieces_->n_pieces()) return true;
    JsonGrammar g = grammar_;
    for (unsigned char c : pieces_->piece(t))
        if (!g.feed(c)) return false;
    return true;
}

void JsonTokenConstraint::commit(tok::TokenId t) {
    if (t < 0 || static_cast<std::uint32_t>(t) >= pieces_->n_pieces()) return;
    for (unsigned char c : pieces_->piece(t)) grammar_.feed(c);
}

bool JsonTokenConstraint::allow_mask(std::uint32_t vocab, std::uint32_t* words) const {
    pieces_->build(grammar_, vocab, words);
    return true;
}

}  // namespace locus::model
