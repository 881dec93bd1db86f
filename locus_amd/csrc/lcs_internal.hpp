// Internal definitions shared by the sampler kernels and the host dispatch.
#pragma once

#include <stdint.h>

#include "locus_sampler.h"

namespace lcs {

// ---- nucleus slices (multi-workgroup passes) ----
constexpr int kSliceThreads = 256;      // threads per slice workgroup
constexpr int kSliceElems = 32;         // logits held in registers per thread
constexpr uint32_t kSliceMax = kSliceThreads * kSliceElems;  // 8192 per slice
constexpr uint32_t kMaxVocab = 262144;
constexpr uint32_t kMaxSlices = kMaxVocab / kSliceMax;       // 32
constexpr uint32_t kTopMax = 20;        // logprob alternatives per row
constexpr uint32_t kWinCap = 64;        // min-p window entries per slice
constexpr uint32_t kFastHistMax = 4096; // penalty window handled by the sliced path

// ---- sliced path (greedy, min-p window and top-k rows): slice_stats maps
// each (row, slice of <= 8192 logits) to a record, row_fin reduces a row's
// records (lcs_slice.hip) ----
constexpr int kSsThreads = 256;         // threads per slice workgroup
constexpr int kSsElems = 32;            // logits per thread (8 f32 / 4 bf16 16-byte groups)
constexpr uint32_t kSsMax = kSsThreads * kSsElems;          // 8192 per slice
constexpr uint32_t kSsMaxSlices = kMaxVocab / kSsMax;       // 32
constexpr uint32_t kRecsPerRow = 64;    // slice records a row owns in the workspace (sliced path: one per
                                        // slice; wave path: one per wave-slice)
constexpr uint32_t kSsTopKMerge = 2048;  // slices x top_k entries row_fin merges
constexpr int kFinThreads = 256;         // row_fin workgroup

// Slice record (64-bit words): a pass's slice workgroups write it, the pass's
// per-row finalize kernel reads it (the kernel boundary orders the two).
namespace rec {
constexpr uint32_t kHdr = 8;         // header words:
// 0: f32 raw max | u16 window entries << 32 | u16 flags << 48
// 1: f64 sum exp(raw - raw max)
// 2: f32 penalised max | u32 its index (first index of the max)
// 3: f32 penalised max over allowed ids | u32 its index
// 4: u32 allowed ids | u32 top-n entries
// 5: f64 bulk: sum over the slice of exp((p - penalised max) / T), f32 terms
// 6: f64 error bound of word 5 (against the reference's own f64 weights)
// 7: f32 raw logit at word 2's index | f32 raw logit at word 3's index
constexpr uint32_t kTop = kHdr;                    // kTopMax rank keys, ascending
constexpr uint32_t kWin = kTop + kTopMax;          // kWinCap rank keys, ascending
constexpr uint32_t kWinRaw = kWin + kWinCap;       // kWinCap raw logits (f32 in the low half)
constexpr uint32_t kWords64 = (kWinRaw + kWinCap + 7) / 8 * 8;
constexpr uint32_t kWords = 2 * kWords64;          // in uint32 units (workspace sizing)
constexpr uint32_t kFlagWinTrunc = 1u;             // more window entries than kWinCap (top kWinCap kept)
constexpr uint32_t kFlagCandOverflow = 2u;         // more top-n candidates than the slice holds
constexpr uint32_t kFlagWinLost = 4u;              // more window entries than the slice could rank
constexpr uint32_t kFlagPenOverflow = 8u;          // more penalised groups than the slice could take
constexpr uint32_t kFlagExact = 16u;               // the row is resolved on the exact path
}  // namespace rec

// ---- single-workgroup exact path ----
constexpr int kGenThreads = 1024;
constexpr uint32_t kGenBins = 2048;
constexpr uint32_t kGenCap = 2048;
constexpr uint32_t kGenHistCap = 8192;
// inline fallback inside the nucleus finalize kernels (256 threads; the
// LDS block shares the nucleus passes' union, so it stays within 32 KB)
constexpr uint32_t kFbBins = 512;
constexpr uint32_t kFbCap = 512;
constexpr uint32_t kFbHistCap = kFastHistMax;
// inline fallback inside row_fin (256 threads, one workgroup per row): bins
// and list as wide as the general kernel's, so a wide min-p window rarely
// needs a radix narrowing
constexpr uint32_t kFinFbBins = 2048;
constexpr uint32_t kFinFbCap = 2048;

enum RowMode : uint32_t { kModeGreedy = 1, kModeWindow = 2, kModeGeneral = 4, kModeTopK = 8, kModeNucleus = 16 };
constexpr uint32_t kTopKMax = 64;         // top_k served by the sliced path
constexpr uint32_t kTopKMerge = 1024;     // slices x top_k entries the finalize merges

// Which implementation path a row takes; pure function of its parameters.
__host__ __device__ inline uint32_t row_mode(const lcs_params& p, bool masked, uint32_t vocab) {
    if (p.temperature <= 0.0f) return kModeGreedy;
    const bool pen = !(p.repeat_penalty == 1.0f && p.frequency_penalty == 0.0f &&
                       p.presence_penalty == 0.0f);
    const bool pen_ok = !pen || p.repeat_last_n <= kFastHistMax;
    const bool topk = p.top_k > 0 && p.top_k < vocab;
    const uint32_t slices = (vocab + kSsMax - 1) / kSsMax;
    if (topk && !masked && pen_ok && p.top_k <= kTopKMax && p.top_k * slices <= kSsTopKMerge) {
        return kModeTopK;
    }
    if (p.min_p > 0.0f && !masked && !topk && pen_ok) return kModeWindow;
    if (pen_ok) return kModeNucleus;   // incl. top-k rows the sliced top-k path cannot take
    return kModeGeneral;
}

// ---- nucleus path (three slice-parallel passes; see lcs_nucleus.hip) ----
constexpr uint32_t kNucBins = 512;      // histogram bins over the tempered offset
constexpr uint32_t kNucRows = 256;      // rows per nucleus launch (workspace rows)
constexpr uint32_t kNucList = 32768;    // candidates the select pass compacts per row (HBM)
constexpr uint32_t kNucRanges = 4;      // bin ranges a row's decisions can need
constexpr uint32_t kNucSub = 128;       // sub-bins per range in the select pass
constexpr float kNucXFloor = -128.0f;   // offsets below collapse into the last bin
constexpr uint32_t kNucFallback = 1u;   // row state flag: resolve with exact_row
struct NucRange {
    uint32_t b0, b1;   // bins [b0, b1]
    uint32_t c0, cnt;  // candidates before the range, in it
    double m0, m;      // mass before the range, in it
};
struct NucRow {
    float maxl;        // penalised candidate max (pass A)
    float sx;          // bins per unit of -x: a power of two <= kNucBins / -x_lo
    uint32_t n_cand;   // candidates after the constraint
    uint32_t use_mask; // the row's mask allows at least one id
    uint32_t maxi;     // index of maxl (first)
    uint32_t nr;       // ranges planned (pass B)
    uint32_t flags;
    uint32_t list_n;   // candidates compacted (pass C counter)
    double log_z;      // raw log-normaliser (pass A)
    double S;          // sum of the weights (pass B)
    NucRange r[kNucRanges];
};

// ---- device-resident penalty windows (lcs_windows_reserve / _load): per
// slot a header, a ring holding the history's last ids (position i at
// i mod H and i mod H + H, so that any run of at most H positions is
// contiguous) and per slice of the sliced path a bucket of the window's
// counts, one entry per 4-position quad that holds a counted id ----
struct WinHdr {
    uint32_t len;     // history length
    uint32_t win;     // the window W (the rows' repeat_last_n)
    uint32_t vocab;   // the vocabulary the buckets are cut for
    uint32_t slen;    // the slice length they are cut at
    int32_t out_id;   // the id at history position len - W (it leaves the window with the next append)
    uint32_t pad[3];
};
// A row's next slot header, staged by its slice 0 workgroup (which wrote the
// appended id into the ring) and copied into place by row_fin: the slice
// kernel's other workgroups read the header, so it cannot change there.
struct WinStage {
    uint32_t flag;    // 1: copy hdr to wh[slot]
    int32_t slot;
    uint32_t pad[6];
    WinHdr hdr;
};
constexpr uint32_t kWinMax = kFastHistMax;   // largest window a slot holds
constexpr uint32_t kBktCap = kSsMax / 4;     // entries a bucket holds (a slice's quads)
// bucket entry: the quad's index in the slice (bits 0-10), then its 4 counts
// (positions 4q + k) of 13 bits at bits 11 + 13k
__host__ __device__ inline uint32_t bkt_quad(uint64_t e) { return (uint32_t)(e & 2047u); }
__host__ __device__ inline uint32_t bkt_count(uint64_t e, uint32_t k) { return (uint32_t)(e >> (11u + 13u * k)) & 8191u; }
__host__ __device__ inline uint64_t bkt_one(uint32_t k) { return 1ull << (11u + 13u * k); }

struct SampleArgs {   // (at most 128 dwords: kernels stage it in LDS, two dwords per lane)
    const void* logits;
    uint64_t row_stride;
    uint32_t rows, vocab, dtype, flags, n_top, mask_words;
    const lcs_params* params;
    const uint32_t* hist_off;
    const int32_t* hist_ids;
    const double* u;
    const uint32_t* mask;
    const uint8_t* has_mask;
    const int32_t* lp_ids;
    int32_t* ids;
    float* chosen_lp;
    int32_t* top_ids;
    float* top_lp;
    lcs_row_diag* diag;
    // workspace
    uint32_t* recs;          // nucleus: rows x slices x rec::kWords
    uint64_t* srecs;         // sliced and wave paths: rows x kRecsPerRow x rec::kWords64
    uint32_t ss_slices;      // sliced path: slices per row (<= kSsMaxSlices)
    uint32_t ss_len;         // sliced path: elements per slice (multiple of 8, <= kSsMax)
    uint32_t* d_ids;         // rows x max_hist (distinct penalised ids)
    float* d_raw;
    float* d_pen;
    uint32_t max_hist;
    uint32_t* status;        // device error word (sticky bits)
    uint32_t slices;         // nucleus: workgroups per row
    uint32_t slice_len;      // nucleus: elements per slice (multiple of 8)
    uint32_t all_sliced;     // 1: the host saw every row take a sliced mode
    uint32_t ss_modes;       // sliced modes the host saw (0: unknown)
    uint32_t all_nucleus;    // 1: the host saw every row take the nucleus mode
    uint32_t nuc_row0;       // first row of this nucleus launch
    // nucleus path workspace, for rows nuc_row0 .. nuc_row0 + kNucRows - 1
    NucRow* nrow;            // kNucRows
    uint64_t* nh_pk;         // kNucRows x kMaxSlices x kNucBins packed bin words (count << 50 + mass)
    uint64_t* nlist;         // kNucRows x kNucList rank keys
    // device-resident penalty windows
    const int32_t* win_slot; // rows: slot, or -1 (NULL: none)
    const int32_t* win_push; // rows: id appended before this call
    const uint32_t* win_len; // rows: history length after the push
    WinHdr* wh;              // slots
    int32_t* wring;          // slots x 2 wring_h
    uint64_t* wbkt;          // slots x kSsMaxSlices x (kBktCap + 1): word 0 the count, then entries
    uint32_t wring_h;        // H: ring half (a power of two above kWinMax)
    WinStage* wstage;        // rows
    const lcs_row_stats* raw_stats;   // rows, or NULL: the rows' raw log-normalisers (lcs_lmhead)
};


struct VerifyArgs {
    const void* logits;
    uint64_t row_stride;
    uint32_t n_seq, rows_per_seq, vocab, dtype;
    const int32_t* draft;
    int32_t* argmax_ids;
    float* draft_lp;
    uint32_t* accept_len;
};

// n-gram drafts (lcs_draft.hip)
constexpr uint32_t kDraftMaxNgram = 64;
constexpr uint32_t kDraftMaxLen = 256;
constexpr uint32_t kNoDraft = 0xffffffffu;
struct DraftArgs {
    uint32_t n_seq, ngram, max_draft;
    const uint32_t* ctx_off;
    const int32_t* ctx_ids;
    int32_t* draft;
    uint32_t* draft_len;
};

// lm-head product with the first statistics in its epilogue (lcs_lmhead.hip)
constexpr uint32_t kLmRows = 64;    // rows per product launch (4 MFMA row tiles)
constexpr uint32_t kLmColsMin = 256;  // vocabulary columns per workgroup (one record block): 256 or 320
struct LmRec {                      // per (row, block of columns)
    float max;                      // the block's largest logit
    uint32_t idx;                   // its first column; bit 31: the block holds the row's draft token
    float sum;                      // sum of exp(logit - max) over the block
    float draft;                    // the draft token's logit (when bit 31 of idx is set)
};
constexpr uint32_t kLmDraftBit = 0x80000000u;
struct LmArgs {
    const uint16_t* x;              // rows x hidden bf16
    const uint16_t* w;              // vocab x hidden bf16
    uint32_t rows, vocab, hidden, m0, nblocks, rows_per_seq;
    uint32_t cols;                  // columns per block (lmhead_cols)
    uint32_t nchunks;               // 64-row chunks of one launch (see lmhead_kernel)
    uint64_t ld_logits;             // elements between logits rows
    const int32_t* draft;
    float* logits;
    int32_t* argmax_ids;
    float* log_z;
    float* draft_lp;
    uint32_t* accept_len;
    LmRec* recs;                    // rows x nblocks
    lcs_row_stats* stats;           // rows, or NULL
};

// status bits
constexpr uint32_t kStatusHistCap = 1u;   // a penalty window exceeded the capacity
constexpr uint32_t kStatusBinCap = 2u;    // selection could not narrow a bin (unexpected)
constexpr uint32_t kStatusWindow = 4u;    // a device-resident window did not match its row

}  // namespace lcs
