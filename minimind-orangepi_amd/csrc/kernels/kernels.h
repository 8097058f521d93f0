// kernels.h -- host-side launch interface of the gfx950 kernels.
//
// Every launcher takes plain device pointers and an explicit stream, performs
// no allocation and no synchronisation, and is therefore safe to record into a
// hipGraph.  Shape checks live in the callers (C-ABI layer and LanguageModel).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mmr {

// -------------------------------------------------------------- L2 warming ----
// A later kernel's reads, described by the blocks that make them.  The
// reading grid has units_x x units_y blocks (x fastest: block (x, y) has id
// x + y * units_x); block (x, y) reads rows [x * rows, (x + 1) * rows) of a
// row-major region (row_bytes apart), bytes [y * seg_bytes, (y + 1) *
// seg_bytes) of each row (seg_bytes = row_bytes: whole rows), never past
// `bytes`.  The dispatcher deals a grid's blocks round-robin over the 8 XCDs
// (block id i on XCD i % 8), each XCD has its own L2, and L2 contents outlive
// a kernel boundary; so blocks of an earlier kernel on XCD x that load what
// the later kernel's blocks on XCD x will read turn those loads into L2 hits.
// A GEMV block reads whole rows (units_y = 1); a split-K GEMM block one K
// chunk of 64 rows.
constexpr int kXcds = 8;
constexpr int kL2WarmRegions = 3;
struct L2Warm {
  const void* base = nullptr;  // nullptr: region unused
  uint32_t bytes = 0;          // region size (byte offsets are 32-bit)
  uint32_t row_bytes = 0;      // multiple of 16
  uint32_t seg_bytes = 0;      // multiple of 16, <= row_bytes
  int rows = 0;                // rows per block
  int units_x = 0, units_y = 1;
};
// Regions and the number of warming blocks that load them (a multiple of
// kXcds; 0 = none).  A kernel that takes an L2WarmSet launches that many
// extra blocks past its own grid (rounded up to a multiple of kXcds).
struct L2WarmSet {
  L2Warm region[kL2WarmRegions];
  int blocks = 0;
};

// ---------------------------------------------------------------- GEMV ----
// y = W x with W fp16 row-major [rows][k] (weights streamed from HBM once),
// x/y fp32, fp32 accumulation.
enum GemvPrologue : int {
  kProPlain = 0,       // x used as given
  kProRmsNorm = 1,     // x := x * (scale * norm_w)      decoder_layer.cpp:32-42
  kProRmsNormFinal = 2,// x := (x * scale) * norm_w      language_model.cpp:24-38
  kProEmbedRmsNorm = 3,// x := embed[seq[*pos]] (fp16 -> fp32), then kProRmsNorm;
                       //      block 0 also stores the raw row to h_out
  kProAttnCombine = 4  // x := log-sum-exp combine of the attention split partials
                       //      (part, splits, hq, hkv, head_dim; k = hq * head_dim)
};
// kProAttnCombine limits: splits <= 16, hq <= 16, k = hq * head_dim <= 1024.
constexpr int kCombineMaxSplits = 16;
constexpr int kCombineMaxHeads = 16;
constexpr int kCombineMaxDim = 1024;

enum GemvEpilogue : int {
  kEpiStore = 0,     // y[r] = dot
  kEpiResidual = 1,  // y[r] = residual[r] + dot
  kEpiSwiGlu = 2,    // rows interleaved (gate_0, up_0, gate_1, up_1, ...):
                     //   y[i] = silu(gate_i) * up_i      decoder_layer.cpp:175-182
  kEpiArgmax = 3     // y[r] = dot (optional); per-block (max, first index) partials,
                     //   reduced by launch_argmax_finalize
};

struct GemvArgs {
  const __half* w = nullptr;
  int rows = 0;
  int k = 0;
  const float* x = nullptr;
  const __half* x_half = nullptr;  // instead of x: fp16 activations (plain and RMSNorm prologues)
  const float* norm_w = nullptr;
  float eps = 0.0f;
  // kProEmbedRmsNorm
  const __half* embed = nullptr;
  const int32_t* seq = nullptr;
  const int32_t* pos = nullptr;
  int vocab = 0;
  float* h_out = nullptr;
  // outputs
  float* y = nullptr;
  const float* residual = nullptr;
  // kProAttnCombine
  const float* part = nullptr;
  int splits = 0, hq = 0, hkv = 0, head_dim = 0;
  // kEpiArgmax: one (value, index) pair per block
  float* part_val = nullptr;
  int* part_idx = nullptr;
  // kProEmbedRmsNorm inside a replayed group of decode steps: when prev_val is
  // set and *pos >= *prompt_len, the token is the argmax of the previous
  // step's lm_head partials (prev_parts <= kGemvMaxPrevParts pairs, first
  // index among equal maxima) instead of seq[*pos], and block 0 stores it to
  // seq_out[*pos] (if *pos < seq_len; seq_out is seq): the argmax finalize's
  // work, done where the token is consumed.
  const float* prev_val = nullptr;
  const int* prev_idx = nullptr;
  int prev_parts = 0;
  const int32_t* prompt_len = nullptr;
  int32_t* seq_out = nullptr;
  int seq_len = 0;
  // kEpiArgmax: block 0 advances *advance_pos by one (the finalize's position
  // bookkeeping, for a step whose finalize is folded into the next step).
  int32_t* advance_pos = nullptr;
};
constexpr int kGemvMaxPrevParts = 2048;

// Reduces the per-block argmax partials (first index among equal maxima),
// writes the token, and optionally does the decode-step bookkeeping: the step
// at position p = *pos writes its prediction to seq[p + 1] when
// p + 1 >= *prompt_len, then advances *pos.  One block.
struct ArgmaxFinalizeArgs {
  const float* part_val = nullptr;
  const int* part_idx = nullptr;
  int parts = 0;
  int32_t* token_out = nullptr;
  int32_t* seq = nullptr;
  int32_t* pos = nullptr;
  const int32_t* prompt_len = nullptr;
  int seq_len = 0;
};
hipError_t launch_argmax_finalize(const ArgmaxFinalizeArgs& a, hipStream_t stream);

struct GemvPlan {
  int lanes_per_row = 32;  // 16, 32 or 64
  int rows_per_group = 1;  // 1, 2 or 4 (even for kEpiSwiGlu)
  int chunks_per_lane = 3; // 16-byte chunks of a row per lane
  int blocks = 0;
};

// Picks a launch shape; lanes_per_row / rows_per_group of 0 mean "auto".
// Returns false when k is not a multiple of 8 or exceeds the supported range.
bool gemv_plan(int rows, int k, GemvEpilogue epi, int lanes_per_row, int rows_per_group, GemvPlan* plan);
hipError_t launch_gemv(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, const GemvPlan& plan,
                       hipStream_t stream);
constexpr int kGemvBlock = 256;

// ------------------------------------------------------------ KV pages ----
// A KV page holds 64 tokens of one layer's keys (or values) for every KV head,
// [Hkv][kKvPage][D]: one head's 64 rows are one contiguous run, and every
// attention tile (64 or 32 tokens, aligned) lies inside one page.
//
// Single-sequence caches keep their pages in segments that double: segment 0
// holds tokens [0, 512), segment s >= 1 tokens [512 << (s - 1), 512 << s).
// A segment's pages are contiguous, so token t's row is found by arithmetic
// (segment from t, then the page and row inside it), with no table read, and
// a cache grows by adding segments without moving a row.  Kernels take the
// segment base pointers as arguments (KvSegs).  The batch path maps pages of
// one pool through per-sequence page tables instead (AttnArgs::page_table).
constexpr int kKvPage = 64;      // tokens per KV page (a multiple of every attention tile)
constexpr int kKvSegShift = 9;   // segment 0 holds 1 << 9 = 512 tokens (8 pages)
constexpr int kKvSegments = 12;  // segments 0..11: up to 512 << 11 = 1,048,576 tokens
struct KvSeg {
  void* k = nullptr;  // [pages][Hkv][kKvPage][D], keys
  void* v = nullptr;  // values, same layout (adjacent to k: one scalar load fetches both)
};
struct KvSegs {
  KvSeg s[kKvSegments];  // unbacked segments are null
};
// Segment holding token t (clamped to the table, so a lookahead past the
// last segment stays in range), its first token, and its size in tokens.
__host__ __device__ constexpr int kv_segment(int t) {
  const unsigned q = static_cast<unsigned>(t) >> kKvSegShift;
  const int s = q == 0 ? 0 : 32 - __builtin_clz(q);
  return s < kKvSegments ? s : kKvSegments - 1;
}
__host__ __device__ constexpr int kv_segment_first(int s) { return s == 0 ? 0 : 1 << (kKvSegShift + s - 1); }
__host__ __device__ constexpr int kv_segment_tokens(int s) {
  return s == 0 ? 1 << kKvSegShift : 1 << (kKvSegShift + s - 1);
}
// Element offset of token t's row for KV head g inside segment s (t in s).
__host__ __device__ constexpr int64_t kv_segment_offset(int s, int t, int g, int hkv, int d) {
  const int r = t - kv_segment_first(s);
  return (static_cast<int64_t>(r / kKvPage) * hkv + g) * kKvPage * d + static_cast<int64_t>(r % kKvPage) * d;
}

// ----------------------------------------------------------- attention ----
// GQA decode attention for one query token over a resident KV cache
// (segmented pages, or a page pool with page tables for a batch), split along
// the context into `splits` tile sets per KV head; the partials are merged by
// a log-sum-exp combine in the consumer.
enum AttnMode : int {
  kAttnFused = 0,     // q/k RMSNorm + RoPE from the raw projection, append k/v at
                      // index *pos, attend over *pos + 1 keys
  kAttnFromCache = 1  // q given (already normalised/rotated), attend over `tokens` keys
};

enum KvDtype : int { kKvF16 = 0, kKvF32 = 1 };

struct AttnArgs {
  const float* qkv = nullptr;       // fused: raw projection [Hq*D + 2*Hkv*D]
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  float eps = 0.0f;
  const float* inv_freq = nullptr;  // fused: [D/2] RoPE frequencies
  const int32_t* pos = nullptr;     // fused: index of the new token (device)
  const float* q = nullptr;         // from-cache: [Hq*D]
  int tokens = 0;                   // from-cache: cached keys
  void* kcache = nullptr;           // batch: page pools (see page_table)
  void* vcache = nullptr;
  int capacity = 0;                 // usable positions (all backed)
  int rows = 0;                     // backed rows per sequence (a multiple of kKvPage)
  int hq = 0, hkv = 0, d = 0;
  int splits = 1;
  float* part = nullptr;            // o [Hkv][splits][R][D], then (m, l) [Hkv][splits][R][2]
  int32_t* err = nullptr;           // set to 1 when *pos is out of range
  // Batch of sequences (grid z): sequence b reads qkv + b * qkv_stride and
  // pos[b], writes part + b * part_stride.
  int batch = 1;
  int64_t qkv_stride = 0;
  int64_t part_stride = 0;
  // Fused mode: the projection may arrive as qkv_parts split-K partials,
  // partial p of sequence b at qkv + p * qkv_part_stride + b * qkv_stride
  // (summed in order; 1 = a plain row).
  int qkv_parts = 1;
  int64_t qkv_part_stride = 0;
  // Batch (fused mode): kcache / vcache are page pools
  // [page][Hkv][kKvPage][D]; page_table[b * pages_per_seq + t / kKvPage] is
  // the page of sequence b's token t; rows = pages_per_seq * kKvPage.
  const int32_t* page_table = nullptr;
  int pages_per_seq = 0;
  // > 0: the table holds page_table[b * pages_per_seq + i] = i *
  // page_interleave + b for every entry, and the kernels apply that rule
  // instead of reading it (one dependent memory access fewer before the
  // first K/V load).
  int page_interleave = 0;
  // Single-sequence fused launches on the per-head kernel: warming blocks past
  // the head blocks load these regions into the XCDs' L2s while the head
  // blocks run.  Other launch shapes ignore them.
  L2WarmSet warm;
  // Single sequence: the cache's segments.  Last, so that the fields every
  // block reads first share the leading kernel-argument cache lines (measured:
  // the table placed after `tokens` cost 6 us per MiniMind2 step).
  KvSegs seg;
};

constexpr int kAttnMaxGroup = 8;  // Hq / Hkv supported
// QKV split-K partials the paged attention prologue sums: at most
// kAttnMaxQkvParts, and a lighter variant for at most kAttnFewQkvParts (the
// batched step asks for that many where 256-column K chunks reach: MiniMind2
// at B = 32, 256 -> 4096 positions, 3 parts against 8: p50 step 0.751 against
// 0.764 ms, 4 parts 0.757, same box).
constexpr int kAttnMaxQkvParts = 8;
constexpr int kAttnFewQkvParts = 3;
size_t attention_partial_floats(int hq, int hkv, int d, int splits);
int attention_tile_tokens(int d);
bool attention_supported(int hq, int hkv, int d);
hipError_t launch_attention(const AttnArgs& a, AttnMode mode, KvDtype kv, hipStream_t stream);
// Merge the split partials into out [Hq*D] (one block per query head and
// 16-dimension slice).  `warm` (one sequence only): warming blocks past the
// merge blocks (see L2WarmSet).
hipError_t launch_attention_combine(const float* part, int hq, int hkv, int d, int splits, float* out,
                                    hipStream_t stream, int batch = 1, int64_t part_stride = 0,
                                    const L2WarmSet* warm = nullptr);

// qkv post-process as a standalone op (reference K2): per-head q/k RMSNorm +
// RoPE at `position`, q -> query_out, k/v appended at cache index `index`.
struct QkvPostArgs {
  const float* qkv = nullptr;
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  float eps = 0.0f;
  const float* inv_freq = nullptr;  // [D/2]
  int position = 0;
  int index = 0;  // cache row the key / value go to (backed)
  KvSegs seg;
  int hq = 0, hkv = 0, d = 0;
  float* query_out = nullptr;
};
hipError_t launch_qkv_postprocess(const QkvPostArgs& a, KvDtype kv, hipStream_t stream);

// ------------------------------------------------------------- prefill ----
// C[m][n] = (residual[m][n] +) sum_k A[m][k] * W[n][k]: A fp32 (row stride
// lda), W fp16 row-major [n][k], C fp32 (row stride ldc); residual may alias
// C.  fp32 matrix cores, fp32 accumulation.  k % 8 == 0, lda % 4 == 0.
// A [rows][cols] as the GEMM's fp16 matrix cores take it: per row and
// `chunk`-wide column chunk a power-of-two scale s (the chunk's max |a|
// mapped into [2^14, 2^15)), hi = fp16(s a), lo = fp16(s a - hi), inv = 1 / s.
// Written once by the kernel producing A, staged by every GEMM block.
// kSplitChunk (one scale per GEMM K tile) is staged as is; kSplitChunkFine
// suits producers that see 32 columns at a time (attention heads, the SwiGLU
// epilogue) and is brought to one scale per K tile while staging.
constexpr int kSplitChunk = 128;
constexpr int kSplitChunkFine = 32;
struct SplitPlanes {
  uint16_t* hi = nullptr;  // [rows][row stride] fp16 bits, cols used
  uint16_t* lo = nullptr;
  float* inv = nullptr;    // [rows][ceil(cols / chunk)], dense
  int chunk = kSplitChunk;
};

struct GemmArgs {
  const float* a = nullptr;
  int lda = 0;
  const __half* w = nullptr;
  const float* residual = nullptr;
  float* c = nullptr;
  int ldc = 0;
  int m = 0, n = 0, k = 0;
  // Split-K: k_splits > 1 writes k_splits partial products (no residual),
  // split z to c + z * split_stride, over its contiguous range of K tiles.
  int k_splits = 1;
  int64_t split_stride = 0;
  // SwiGLU epilogue over interleaved gate/up columns: c receives
  // act[m][n / 2] (row stride ldc); needs k_splits == 1 and no residual.
  bool swiglu = false;
  // A given pre-split instead of `a` (SplitPlanes): fp16 bit planes hi and lo
  // [m][lda] and inv [m][ceil(k / a_chunk)]; a_chunk kSplitChunkFine only
  // for the plain store (no residual, no SwiGLU).
  const uint16_t* a_hi = nullptr;
  const uint16_t* a_lo = nullptr;
  const float* a_inv = nullptr;
  int a_chunk = kSplitChunk;
  // Keep the call on the register-staged kernel even where the direct-to-LDS
  // one applies (both compute the full product; a comparison switch).
  bool register_staged = false;
  // SwiGLU epilogue only: act as SplitPlanes instead of into c (c unused),
  // with kSplitChunkFine chunks (planes [m][ldc], inv [m][n / 2 / 32]);
  // needs the tiling gemm_swiglu_split_supported accepts.
  SplitPlanes act_split;
};
bool gemm_supported(int m, int n, int k);
// Split count launch_gemm accepts and uses well for this shape: about four
// 128-wide K tiles per split; 1 where the few-rows path applies.
int gemm_k_splits(int m, int n, int k);
// Whether launch_gemm takes the SwiGLU epilogue for this shape (unsplit tiles).
bool gemm_swiglu_supported(int m, int n, int k);
// Whether launch_gemm takes pre-split A (a_hi / a_lo / a_inv) for this shape
// (the tiled path; the few-rows path reads fp32 A).
bool gemm_presplit_supported(int m, int n, int k);
// Whether the SwiGLU epilogue can write act pre-split (act_split) for this
// shape: unsplit tiles 64 wide or wider (64 x 128, 64 x 64 or 32 x 64: a block holds
// whole 32-column act chunks of its rows) and
// n a multiple of 64.
bool gemm_swiglu_split_supported(int m, int n, int k);
hipError_t launch_gemm(const GemmArgs& g, hipStream_t stream);

// Rows of the fused qkv projection for tokens at positions start ..
// start + tokens - 1: per-head q/k RMSNorm + RoPE, q -> query rows, k/v
// written to cache rows row0 .. row0 + tokens - 1 (row0 = start when cache
// rows are positions).
struct QkvRowsArgs {
  const float* qkv = nullptr;  // [tokens][qkv_stride]
  int qkv_stride = 0;
  // Split-K partials of the projection: qkv holds qkv_parts (<= kQkvRowsMaxParts)
  // sets qkv_part_stride floats apart, added in split order.
  int qkv_parts = 1;
  int64_t qkv_part_stride = 0;
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  float eps = 0.0f;
  const float* inv_freq = nullptr;  // [D/2]
  int start = 0;  // RoPE position of token 0
  int row0 = 0;   // cache row of token 0
  int tokens = 0;
  KvSegs seg;  // rows row0 .. row0 + tokens - 1 backed
  int hq = 0, hkv = 0, d = 0;
  float* query = nullptr;  // [tokens][query_stride]
  int query_stride = 0;
};
constexpr int kQkvRowsMaxParts = 4;
hipError_t launch_qkv_rows(const QkvRowsArgs& a, KvDtype kv, hipStream_t stream);

// Causal attention of query rows at positions start .. start + tokens - 1
// over cache keys 0 .. each query's position.
struct PrefillAttnArgs {
  const float* query = nullptr;  // [tokens][query_stride], normalised + rotated
  int query_stride = 0;
  KvSegs seg;  // rows 0 .. start + tokens - 1 backed
  int start = 0;
  int tokens = 0;
  int hq = 0, hkv = 0, d = 0;
  float* out = nullptr;  // [tokens][out_stride]; may be null when out_split is set
  int out_stride = 0;
  // Optional: the output also as SplitPlanes with kSplitChunkFine chunks,
  // planes [tokens][out_stride], inv [tokens][hq d / 32]; needs d % 32 == 0.
  SplitPlanes out_split;
};
hipError_t launch_prefill_attention(const PrefillAttnArgs& a, KvDtype kv, hipStream_t stream);

// --------------------------------------------------------------- batch ----
// Decode of a batch of independent sequences, sequence b at its own device
// position pos[b] with its tokens in seq[b * seq_stride ..].
// h[b][:] = embed[seq[b][pos[b]]] (fp16 -> fp32); out-of-range ids are clamped
// (the host validates every id it uploads).
hipError_t launch_batch_embed(const __half* embed, const int32_t* seq, int seq_stride, const int32_t* pos, int batch,
                              int vocab, int hidden, float* h, hipStream_t stream);
// Per sequence: first index of the maximum of logits[b][:vocab]; token_out[b]
// receives it, and the step bookkeeping of launch_argmax_finalize runs per
// sequence (seq[b][p + 1] when p + 1 >= prompt_len[b], then pos[b] = p + 1).
hipError_t launch_batch_argmax(const float* logits, int vocab, int batch, int32_t* token_out, int32_t* seq,
                               int seq_stride, int32_t* pos, const int32_t* prompt_len, int seq_len,
                               hipStream_t stream);

// Split-K projection for few rows (batched decode): part[s][m][n] =
// sum over k in [s kc, (s + 1) kc) of a[m][k] * w[n][k]; consumers sum the
// splits in order.  m <= 32, k % 32 == 0, kc a multiple of 32 <= 256.
struct SplitKArgs {
  const float* a = nullptr;
  int lda = 0;
  const __half* w = nullptr;
  float* part = nullptr;
  int m = 0, n = 0, k = 0;
  int kc = 0;
  // SwiGLU input: when gu is set, A[r][j] = silu(g) * u with g, u the sums (in
  // split order) of gu[s][r][2j] and gu[s][r][2j + 1] over s < gu_splits
  // (the gate_up partials, [gu_splits][m][2k]); a and lda are unused.
  const float* gu = nullptr;
  int gu_splits = 0;
  // Attention-combine input: when attn_part is set, row r of A is sequence
  // r's attention output merged from its split partials (the layout of
  // attn_o_offset / attn_ml_offset, attn_splits splits, attn_part_stride
  // floats per sequence); a, lda and gu are unused.
  const float* attn_part = nullptr;
  int attn_splits = 0;
  int64_t attn_part_stride = 0;
  int hq = 0, hkv = 0, d = 0;
};
// W rows per split-K block: the launch grid is (ceil(n / kSplitKRows), k / kc).
constexpr int kSplitKRows = 64;
// (W row block, K chunk) of split-K block `block` (linear id x + row_blocks y
// of the grid (row_blocks, chunks)).  The blocks of one K chunk stage the same
// A rows (or the same partials); block b runs on XCD b mod kXcds, so with the
// chunk count a multiple of kXcds, XCD x takes every row block of chunks
// x * chunks / kXcds .. and each chunk's A is fetched into one L2.  Otherwise
// block b takes (b mod row_blocks, b / row_blocks).  Every pair is taken by
// exactly one block.
struct SplitKTile {
  int row_block, chunk;
};
__host__ __device__ inline SplitKTile splitk_block_tile(int block, int row_blocks, int chunks) {
  if (chunks % kXcds != 0) return SplitKTile{block % row_blocks, block / row_blocks};
  const int slot = block / kXcds;
  return SplitKTile{slot % row_blocks, (block % kXcds) * (chunks / kXcds) + slot / row_blocks};
}
// K chunk (a multiple of 32 that divides k, at most 256; 0 when k is not a
// multiple of 32); splits = k / kc.
int splitk_chunk(int n, int k);
// Whether launch_gemm_splitk takes SwiGLU input for m rows, chunk kc and
// gu_splits gate_up partials (the staging loads must fit in registers).
bool splitk_swiglu_supported(int m, int kc, int gu_splits);
// Whether launch_gemm_splitk takes attention-combine input for m rows, chunk
// kc, attn_splits splits and head_dim d.
bool splitk_combine_supported(int m, int kc, int attn_splits, int d);
hipError_t launch_gemm_splitk(const SplitKArgs& g, hipStream_t stream);
// h[b] += sum_s part[s][b] (splits may be 0), x[b] = RMSNorm(h[b]); x may be
// null when `split` receives the normalised rows instead (or as well).
// `warm`: warming blocks past the batch rows (see L2WarmSet).
hipError_t launch_batch_residual_norm(float* h, const float* part, int splits, int batch, int cols, const float* w,
                                      float eps, float* x, bool final_norm, hipStream_t stream,
                                      const SplitPlanes* split = nullptr, const L2WarmSet* warm = nullptr);
// act[b][i] = silu(sum_s part[s][b][2i]) * sum_s part[s][b][2i + 1].
hipError_t launch_batch_swiglu(const float* part, int splits, int batch, int f, float* act, hipStream_t stream);
// out[b][i] = sum_s part[s][b][i].
hipError_t launch_batch_sum_parts(const float* part, int splits, int batch, int n, float* out, hipStream_t stream);
// logits[b] = sum_s part[s][b] (lm_head split-K partials), then the batch
// argmax with its bookkeeping (one kernel for up to 4 partials).
hipError_t launch_batch_head(const float* part, int splits, int vocab, int batch, float* logits, int32_t* token_out,
                             int32_t* seq, int seq_stride, int32_t* pos, const int32_t* prompt_len, int seq_len,
                             hipStream_t stream);

// -------------------------------------------------------- small models ----
// A whole decode step in one workgroup (tiny.hip) for models whose shapes the
// GEMV / attention kernels do not take (the reference's toy model: hidden 4,
// head_dim 2).  Same step bookkeeping as launch_argmax_finalize.
struct TinyLayerPtrs {
  const float* input_norm = nullptr;
  const float* post_norm = nullptr;
  const float* q_norm = nullptr;
  const float* k_norm = nullptr;
  const __half* qkv = nullptr;      // [(Hq + 2 Hkv) d][H]
  const __half* o = nullptr;        // [H][Hq d]
  const __half* gate_up = nullptr;  // [2F][H] interleaved gate/up rows
  const __half* down = nullptr;     // [H][F]
  void* kcache = nullptr;           // [Hkv][rows][d]
  void* vcache = nullptr;
};
struct TinyStepArgs {
  const __half* embed = nullptr;    // [V][H]
  const __half* lm_head = nullptr;  // [V][H]
  const float* final_norm = nullptr;
  const TinyLayerPtrs* layers = nullptr;  // device array [n_layers]
  int n_layers = 0;
  const float* inv_freq = nullptr;  // [d/2]
  int hidden = 0, hq = 0, hkv = 0, d = 0, f = 0, vocab = 0;
  float eps = 0.0f;
  int rows = 0;      // cache rows per KV head
  int capacity = 0;  // usable positions
  int32_t* seq = nullptr;
  int32_t* pos = nullptr;
  const int32_t* prompt_len = nullptr;
  int seq_len = 0;
  int32_t* err = nullptr;
  int32_t* token_out = nullptr;
  float* logits = nullptr;  // [V]
};
constexpr int kTinyMaxWidth = 1024;   // hidden and (Hq + 2 Hkv) d
constexpr int kTinyMaxFfn = 2048;
constexpr int kTinyMaxHeadDim = 128;  // even
constexpr int kTinyMaxContext = 2048; // positions of one state
bool tiny_step_supported(int hidden, int hq, int hkv, int d, int f, int vocab, int capacity);
hipError_t launch_tiny_step(const TinyStepArgs& a, KvDtype kv, hipStream_t stream);

// ------------------------------------------------------------- support ----
hipError_t launch_rms_norm_rows(const float* in, const float* w, float eps, int rows, int cols, float* out,
                                hipStream_t stream, bool final_norm = false);
hipError_t launch_add(const float* a, const float* b, int64_t n, float* out, hipStream_t stream);
hipError_t launch_swiglu_rows(const float* gate_up, int rows, int cols, float* out, hipStream_t stream);
hipError_t launch_embedding_gather(const __half* table, const int32_t* ids, int tokens, int vocab, int hidden,
                                   float* out, int32_t* err, hipStream_t stream);

// Per-kernel time of a hipGraph chain of `kernels` trivial launches of
// `blocks` x 256 threads (empty, or one dependent load + store), replayed
// `reps` times on a private stream (probe.hip).
hipError_t measure_launch_floor(int kernels, int blocks, bool load_store, int reps, float* us_per_kernel);

}  // namespace mmr
