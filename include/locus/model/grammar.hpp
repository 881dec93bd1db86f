/*
 * JSON constrained decoding on the host: the incremental validator of the
 * reference (JsonGrammar, src/locus/model/grammar.hpp:24-57, grammar.cpp),
 * the per-token constraint of its server (JsonTokenConstraint,
 * src/locus/server/server.cpp:154-185), and a bitmask builder that produces
 * the V/32 allow words the GPU sampler consumes.
 *
 * JsonGrammar accepts exactly the byte sequences the reference's accepts:
 * objects, arrays, strings (escapes, \uXXXX), keywords checked exactly,
 * numbers leniently (digits and . e E + -), a number ended by re-reading its
 * delimiter. Its state is a few bytes plus the container stack, and one
 * feed() can be undone in O(1) (mark()/undo()), which the mask builder uses
 * to walk a byte trie of the vocabulary instead of copying the grammar once
 * per token.
 */
#pragma once

#include <cstdint>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "locus/model/sampling.hpp"

namespace locus::model {

class JsonGrammar {
  public:
    /** Advances on byte b; false if b cannot continue a valid JSON value
     * (a rejected byte may leave the state changed, as the reference's; a
     * rejected feed is only ever followed by dropping the copy). */
    bool feed(std::uint8_t b);
    /** A complete top-level value has been consumed (trailing whitespace
     * keeps it complete). */
    bool complete() const;

    /** O(1) snapshot of everything one feed() can change. */
    struct Mark {
        std::uint8_t mode, bits, aux, top;
        std::uint32_t depth;
    };
    Mark mark() const;
    void undo(const Mark& m);

    /** Appends a key of the state a byte string of length <= max_len can
     * observe (mode, flags, keyword/escape progress, the top containers). */
    void state_key(std::uint32_t max_len, std::string& key) const;

  private:
    // parser modes (the reference's S, grammar.hpp:35-47)
    enum Mode : std::uint8_t {
        kValue, kArrayOpen, kObjectOpen, kKey, kColon, kString, kEscape, kUnicode,
        kNumber, kKeyword, kDone
    };
    enum : std::uint8_t { kInKey = 1, kNumDigit = 2 };
    bool start_value(std::uint8_t b);
    bool close(char want);

    std::uint8_t mode_ = kValue;
    std::uint8_t bits_ = 0;   // kInKey | kNumDigit
    std::uint8_t aux_ = 0;    // \u digits left, or keyword id << 4 | matched length
    std::string open_;        // '{' / '[' per open container
};

/** Byte trie of a vocabulary's token pieces plus an allow-mask cache keyed by
 * grammar state. Tokens at or beyond the piece table are always allowed and
 * an empty piece is allowed (server.cpp:160-171). Thread-safe. */
class JsonMaskBuilder {
  public:
    explicit JsonMaskBuilder(std::vector<std::string> pieces, std::size_t cache_entries = 256);
    const std::string& piece(tok::TokenId t) const { return pieces_[static_cast<std::size_t>(t)]; }
    std::uint32_t n_pieces() const { return static_cast<std::uint32_t>(pieces_.size()); }
    /** Fills words[ceil(vocab/32)] with the tokens whose bytes g accepts. */
    void build(const JsonGrammar& g, std::uint32_t vocab, std::uint32_t* words) const;
    /** Cache statistics (hits, misses). */
    std::pair<std::uint64_t, std::uint64_t> cache_stats() const;

  private:
    struct Node {
        std::uint32_t child = 0;    // first child (0 = none; node 0 is the root)
        std::uint32_t sibling = 0;  // next sibling
        std::uint32_t tok_begin = 0, tok_end = 0;  // tokens ending here: toks_[begin, end)
        std::uint8_t byte = 0;
    };
    void walk(JsonGrammar g, std::uint32_t vocab, std::uint32_t* words) const;

    std::vector<std::string> pieces_;
    std::vector<Node> nodes_;
    std::vector<tok::TokenId> toks_;
    std::uint32_t max_len_ = 0;
    std::size_t cache_cap_;
    mutable std::mutex mu_;
    mutable std::list<std::pair<std::string, std::vector<std::uint32_t>>> lru_;
    mutable std::unordered_map<std::string, decltype(lru_)::iterator> index_;
    mutable std::uint64_t hits_ = 0, misses_ = 0;
};

/** The reference's JSON-mode constraint (server.cpp:154-185) with allow_mask()
 * served by a shared JsonMaskBuilder. */
class JsonTokenConstraint : public TokenConstraint {
  public:
    explicit JsonTokenConstraint(std::shared_ptr<const JsonMaskBuilder> pieces)
        : pieces_(std::move(pieces)) {}
    bool allows(tok::TokenId t) const override;
    void commit(tok::TokenId t) override;
    bool allow_mask(std::uint32_t vocab, std::uint32_t* words) const override;
    const JsonGrammar& grammar() const { return grammar_; }

  private:
    std::shared_ptr<const JsonMaskBuilder> pieces_;
    JsonGrammar grammar_;
};

}  // namespace locus::model
