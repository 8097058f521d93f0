// attention.hip -- GQA decode attention over a resident KV cache (gfx950).
//
// Replaces, on the decode path:
//  * the QKV post-process + resident KV append (reference K2,
//    mini_mind_decode_qkv_postprocess via device_decode_qkv_postprocess,
//    ascend_custom_ops.cpp:825-884; CPU semantics decoder_layer.cpp:342-359),
//  * the decode attention (reference K3 via device_attention_from_cache,
//    ascend_custom_ops.cpp:886-916; CPU semantics decoder_layer.cpp:184-234).
//
// Layout: per layer the cache holds K and V in 64-token pages
// [kv_head][64][head_dim] (fp16 or fp32): a single sequence's pages sit in
// segments that double in size (KvSegs, token -> row by arithmetic), a
// batch's in one pool behind per-sequence page tables.  Every attention tile
// is one contiguous run of one KV head's rows inside one page.
//
// attention_split_kernel, grid (splits, kv_heads), 256 threads.  Block
// (s, g) owns KV head g and the 64-token tiles s, s + splits, ... (32-token
// tiles for d = 128), and serves all Hq/Hkv query heads of the group from one
// read of K/V.  Latency is the cost, so the first tile's K/V loads, the raw
// q/k/v and the RoPE frequencies are all issued before the device position
// arrives; RoPE angles are float(pos) * inv_freq with inv_freq from the host
// (the reference formula) and cos/sin evaluated on the device.
//   1. q RMSNorm + RoPE in registers (a wave per head, a lane per RoPE
//      pair), then into LDS; the block holding the new token also
//      normalises/rotates its k, rounds k and v to the cache dtype and appends
//      them (fused mode).  The first tile's staging barrier is the only one
//      before the scores;
//   2. per tile: scores q.k / sqrt(d) with one lane per token, online softmax
//      with one wave per query head, P.V with one lane per dimension pair;
//   3. the block writes its (max, sum, o[d]) partial per head; splits with no
//      tile write the neutral partial (-inf, 0, 0).
// No block waits for another: the log-sum-exp combine runs in the consumer
// (the O-projection GEMV prologue, or attention_combine_kernel).
//
// attention_mfma_kernel takes the split kernel's place for an fp16 cache with
// 64-token tiles: same grid, prologue and partials, the scores and P.V on the
// fp16 matrix cores.  attention_head_kernel serves short single-sequence
// contexts (one block per query head and split, L2-warming blocks alongside).
#include <type_traits>

#include "attention_common.h"
#include "device_common.h"
#include "kernels.h"

namespace mmr {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
// Waves per query head in attention_head_kernel's one-head blocks: eight
// (two per SIMD, half a tile's tokens each) where a tile's tokens and a
// head's dims split evenly over them (each wave holds whole tokens, each
// token's lanes whole quads of dims), else four.  Eight against four,
// MiniMind2 at 768 keys: the launch without its warming blocks 3.76 -> 3.70
// us, decode 4,026 -> 4,032 tok/s, 1,024 keys 274.3 -> 271.6 us per step.
constexpr int kHeadWaves = 8;
template <int D, int kHeads>
constexpr int head_kernel_waves() {
  constexpr int TT = attn_tile_tokens<D>();
  constexpr bool fits = TT % kHeadWaves == 0 && kWave % (TT / kHeadWaves) == 0 &&
                        (D / 4) % (kWave / (TT / kHeadWaves)) == 0;
  return kHeads == 1 && fits ? kHeadWaves : kAttnWaves;
}

template <typename KV>
__device__ __forceinline__ void chunk_to_float(const uint4& c, float* dst);
template <>
__device__ __forceinline__ void chunk_to_float<__half>(const uint4& c, float* dst) {
  half8_to_float8(c, dst);
}
template <>
__device__ __forceinline__ void chunk_to_float<float>(const uint4& c, float* dst) {
  dst[0] = __uint_as_float(c.x);
  dst[1] = __uint_as_float(c.y);
  dst[2] = __uint_as_float(c.z);
  dst[3] = __uint_as_float(c.w);
}

// One head in registers, one wave: lane i < d/2 holds the RoPE pair
// (x0 = x[i], x1 = x[i + d/2]) and the gains at the same dims (lanes past d/2
// hold zeros).  Per-head RMSNorm (decoder_layer.cpp:32-42, x * (scale * w)),
// then rotate-half RoPE with the pair's (cos, sin) (decoder_layer.cpp:139-152),
// in place; no LDS and no barrier.
template <int D>
__device__ __forceinline__ void wave_norm_rope_pair(float& x0, float& x1, float w0, float w1, float eps, float c,
                                                    float s) {
  const float ss = group_sum<kWave>(x0 * x0 + x1 * x1);
  // v_rsq_f32 (about 1 ulp) of the mean as one fma with 1 / d (a constant)
  const float scale = __builtin_amdgcn_rsqf(fmaf(ss, 1.0f / static_cast<float>(D), eps));
  const float first = x0 * (scale * w0);
  const float second = x1 * (scale * w1);
  x0 = first * c - second * s;
  x1 = second * c + first * s;
}

// Lane `src` of v, as a wave-uniform value (src a compile-time constant).
__device__ __forceinline__ float lane_value(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

__device__ __forceinline__ void pv_fma(float2& acc, float p, const float2& v) {
  acc.x = fmaf(p, v.x, acc.x);
  acc.y = fmaf(p, v.y, acc.y);
}

// P.V work split: thread = (dimension pair, token group); the largest power of
// two <= 8 groups that fits 256 threads and divides the tile.
template <int D, int TT>
constexpr int attn_pv_groups() {
  int g = 8;
  while (g > 1 && (g * (D / 2) > kAttnThreads || TT % g != 0)) g /= 2;
  return g;
}

// Token t's K and V rows for KV head g.  Single sequence: the segmented
// cache, where page_of(t) is t's segment (arithmetic, no memory access) and
// the row sits at a computed offset in that segment.  Batch: page pools
// [page][Hkv][kKvPage][D] with this sequence's page table mapping t / kKvPage
// to a page.  A tile never crosses a page (tiles are <= kKvPage tokens and
// aligned), so one lookup serves a whole tile.
template <typename KV, int D, bool PAGED>
struct KvRows {
  const AttnArgs& a;
  const int32_t* pages;
  int g, b;
  __device__ __forceinline__ KvRows(const AttnArgs& args, int seq, int group)
      : a(args), pages(args.page_table + static_cast<int64_t>(seq) * args.pages_per_seq), g(group), b(seq) {}
  // Batch: the page holding token t (its index clamped into the page table,
  // so a lookahead past the context stays in range).  With page_interleave the
  // table's own rule is applied without reading it; otherwise the table is
  // read through the constant address space (read-only here, uniform index):
  // a scalar-cache load whose wait (lgkmcnt) never covers the vector K/V
  // loads in flight.  Single sequence: t's segment.
  __device__ __forceinline__ int page_of(int t) const {
    if constexpr (PAGED) {
      const int idx = min(t / kKvPage, a.pages_per_seq - 1);
      if (a.page_interleave > 0) return idx * a.page_interleave + b;
      using ConstTable = const __attribute__((address_space(4))) int32_t;
      return ((ConstTable*)pages)[idx];
    } else {
      return kv_segment(t);
    }
  }
  __device__ __forceinline__ int64_t offset(int page, int t) const {
    if constexpr (PAGED) {
      return ((static_cast<int64_t>(page) * a.hkv + g) * kKvPage + t % kKvPage) * D;
    } else {
      return kv_segment_offset(page, t, g, a.hkv, D);
    }
  }
  __device__ __forceinline__ KV* k_at(int page, int t) const {
    if constexpr (PAGED) {
      return static_cast<KV*>(a.kcache) + offset(page, t);
    } else {
      return static_cast<KV*>(a.seg.s[page].k) + offset(page, t);
    }
  }
  __device__ __forceinline__ KV* v_at(int page, int t) const {
    if constexpr (PAGED) {
      return static_cast<KV*>(a.vcache) + offset(page, t);
    } else {
      return static_cast<KV*>(a.seg.s[page].v) + offset(page, t);
    }
  }
  // Rows of the block's speculative first tile at t_spec when `spec` (it is
  // backed), else of token 0.  Single sequence: the tile's segment pointer is
  // one kernel-argument load at a computed index, issued once the split is
  // known (a scalar round trip after the first argument batch; measured
  // against a cache with one contiguous run per head: +0.2 us per bare
  // launch, no change in the MiniMind2 step at 768 keys, +2% at 4096).
  // Selecting with masks keeps the K/V loads global loads (a pointer select
  // made the compiler fall back to flat loads).
  __device__ __forceinline__ void first_tile(int t_spec, bool spec, const KV*& k, const KV*& v) const {
    if constexpr (PAGED) {
      const int t = spec ? t_spec : 0;
      const int pg = page_of(t);
      k = k_at(pg, t);
      v = v_at(pg, t);
    } else {
      const int sg = kv_segment(t_spec);
      const KvSeg cand = a.seg.s[sg];
      const KvSeg zero = a.seg.s[0];
      // Selected with masks, not a branch: the compiler keeps both pointer
      // loads unconditional instead of sinking them behind the `rows` test.
      const uint64_t take = spec ? ~uint64_t{0} : uint64_t{0};
      const uint64_t off = static_cast<uint64_t>(kv_segment_offset(sg, t_spec, g, a.hkv, D)) & take;  // token 0: g's run
      const uint64_t off0 = static_cast<uint64_t>(kv_segment_offset(0, 0, g, a.hkv, D)) & ~take;
      const uint64_t kb = (reinterpret_cast<uint64_t>(cand.k) & take) | (reinterpret_cast<uint64_t>(zero.k) & ~take);
      const uint64_t vb = (reinterpret_cast<uint64_t>(cand.v) & take) | (reinterpret_cast<uint64_t>(zero.v) & ~take);
      k = reinterpret_cast<const KV*>(kb) + (off | off0);
      v = reinterpret_cast<const KV*>(vb) + (off | off0);
    }
  }
};

template <typename KV, int D, int MODE, bool PAGED, int QP = 1>
__global__ __launch_bounds__(kAttnThreads) void attention_split_kernel(AttnArgs a) {
  constexpr int TT = attn_tile_tokens<D>();
  constexpr int LD = D + 4;  // padded row: conflict-free 16-byte LDS reads
  constexpr int CH = 16 / static_cast<int>(sizeof(KV));
  constexpr int kChunks = TT * D / CH;  // 16-byte chunks per K (or V) tile
  constexpr int kPerThread = (kChunks + kAttnThreads - 1) / kAttnThreads;
  constexpr int kPairs = D / 2;
  constexpr int kPvGroups = attn_pv_groups<D, TT>();
  constexpr int kPvTokens = TT / kPvGroups;
  __shared__ __align__(16) float q_s[kAttnMaxGroup][D];
  __shared__ __align__(16) float k_s[TT][LD];
  __shared__ __align__(16) float v_s[TT][LD];
  __shared__ __align__(16) float p_s[TT][kAttnMaxGroup];  // token-major: one 16-byte read per 4 heads
  __shared__ float alpha_s[kAttnMaxGroup];
  static_assert(kPvGroups * kAttnMaxGroup * D <= TT * LD, "P.V reduction must fit in k_s");
  static_assert(D / 2 <= kWave, "a wave holds one head as d/2 RoPE pairs");

  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int b = blockIdx.z;  // sequence of a batch (0 for a single sequence)
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int R = a.hq / a.hkv;
  const int S = a.splits;
  const KvRows<KV, D, PAGED> kv_rows(a, b, g);
  float* part = a.part + static_cast<int64_t>(b) * a.part_stride;
  const float* qkv_row = a.qkv + static_cast<int64_t>(b) * a.qkv_stride;

  // ---- 1. independent loads, issued before the position is known: the raw
  // q/k/v (every QKV partial), gains and RoPE frequencies first, then the
  // block's first tile.  Vector loads complete in issue order, so the q/k
  // norm and RoPE wait for the first group alone while the tile is still
  // arriving (the partials are summed after the tile's loads are out) ----
  // The position is read through the scalar cache (no kernel writes it while
  // this one runs), so no vector load waits behind its round trip.
  int p = -1;
  if constexpr (MODE == kAttnFused) p = ((const __attribute__((address_space(4))) int32_t*)a.pos)[b];
  // Loads are unconditional (indices clamped into range, values masked
  // afterwards): a predicated load makes the compiler wait for it before the
  // branch joins, which would serialise these round trips.  Lane i < d/2
  // holds dims (i, i + d/2), the pair RoPE rotates together.
  const int d0 = min(lane, D / 2 - 1), d1 = d0 + D / 2;
  const bool in_pair = lane < D / 2;
  // The batched (paged) path may hand the projection over as up to QP
  // split-K partials (QP = kAttnFewQkvParts or kAttnMaxQkvParts): every part's
  // load is issued (part index clamped, parts past qkv_parts weighted 0) and
  // the parts summed in order.
  constexpr int kParts = PAGED ? QP : 1;
  float rq0[kParts][2], rq1[kParts][2], rk0[kParts], rk1[kParts], rv0[kParts], rv1[kParts];
#pragma unroll
  for (int pt = 0; pt < kParts; ++pt) {
    const float* row = qkv_row + static_cast<int64_t>(min(pt, a.qkv_parts - 1)) * a.qkv_part_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int h = min(wave + j * kAttnWaves, R - 1);
      const float* src = (MODE == kAttnFused ? row : a.q) + (g * R + h) * D;
      rq0[pt][j] = src[d0];
      rq1[pt][j] = src[d1];
    }
    rk0[pt] = rk1[pt] = rv0[pt] = rv1[pt] = 0.0f;
    if constexpr (MODE == kAttnFused) {
      const float* kraw = row + a.hq * D + g * D;
      const float* vraw = kraw + a.hkv * D;
      rk0[pt] = kraw[d0];
      rv0[pt] = vraw[d0];
      rk1[pt] = kraw[d1];
      rv1[pt] = vraw[d1];
    }
  }
  float inv_freq = 0.0f, qw0 = 0.0f, qw1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f;
  if constexpr (MODE == kAttnFused) {
    inv_freq = a.inv_freq[d0];
    qw0 = a.q_norm[d0];
    qw1 = a.q_norm[d1];
    kw0 = a.k_norm[d0];
    kw1 = a.k_norm[d1];
  }
  asm volatile("" ::: "memory");  // the loads above go out before the tile's
  uint4 kc[kPerThread], vc[kPerThread];
  const int t_spec = split * TT;
  const bool spec = t_spec + TT <= a.rows;
  const KV* kspec;
  const KV* vspec;
  kv_rows.first_tile(t_spec, spec, kspec, vspec);  // always backed; unused unless spec
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int c = min(static_cast<int>(threadIdx.x) + i * kAttnThreads, kChunks - 1);
    kc[i] = *reinterpret_cast<const uint4*>(kspec + c * CH);
    vc[i] = *reinterpret_cast<const uint4*>(vspec + c * CH);
  }
  // Page of the block's second tile, looked up one tile ahead of its fetch.
  int next_page = kv_rows.page_of((split + S) * TT);
  asm volatile("" ::: "memory");
  float qx0[2] = {0.0f, 0.0f}, qx1[2] = {0.0f, 0.0f};
  float kx0 = 0.0f, kx1 = 0.0f, vx0 = 0.0f, vx1 = 0.0f;
#pragma unroll
  for (int pt = 0; pt < kParts; ++pt) {
    const float wgt = pt < a.qkv_parts ? 1.0f : 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      qx0[j] += wgt * rq0[pt][j];
      qx1[j] += wgt * rq1[pt][j];
    }
    kx0 += wgt * rk0[pt];
    vx0 += wgt * rv0[pt];
    kx1 += wgt * rk1[pt];
    vx1 += wgt * rv1[pt];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    qx0[j] = in_pair ? qx0[j] : 0.0f;
    qx1[j] = in_pair ? qx1[j] : 0.0f;
  }
  kx0 = in_pair ? kx0 : 0.0f;
  vx0 = in_pair ? vx0 : 0.0f;
  kx1 = in_pair ? kx1 : 0.0f;
  vx1 = in_pair ? vx1 : 0.0f;

  // ---- 2. extent of the context ----
  int n_keys;
  if constexpr (MODE == kAttnFused) {
    const bool ok = p >= 0 && p < a.capacity;
    if (!ok && threadIdx.x == 0 && split == 0 && g == 0) *a.err = 1;  // vector store, once per sequence
    n_keys = ok ? p + 1 : 0;
  } else {
    n_keys = a.tokens < a.capacity ? a.tokens : a.capacity;
  }
  const int n_tiles = (n_keys + TT - 1) / TT;

  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.0f, 0.0f};
  // P.V ownership: thread = (dimensions 2 * pv_pair + {0, 1}, token group).
  const int pv_pair = threadIdx.x % kPairs;
  const int pv_group = threadIdx.x / kPairs;
  const bool pv_active = static_cast<int>(threadIdx.x) < kPvGroups * kPairs;
  float2 pacc[kAttnMaxGroup];
#pragma unroll
  for (int h = 0; h < kAttnMaxGroup; ++h) pacc[h] = make_float2(0.0f, 0.0f);

  if (split < n_tiles) {
    // ---- 3. queries (and the new key/value), RoPE angle from the position,
    // all in registers; the first tile's staging barrier publishes q_s ----
    float rc = 1.0f, rs = 0.0f;
    if constexpr (MODE == kAttnFused) {
      if (in_pair) sincosf(static_cast<float>(p) * inv_freq, &rs, &rc);
    }
    // q staged times log2(e) / sqrt(d): the scores come out divided by
    // sqrt(d) (decoder_layer.cpp:213) and in base-2 units for exp2.
    const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(D));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int h = wave + j * kAttnWaves;
      if (h < R) {
        if constexpr (MODE == kAttnFused) wave_norm_rope_pair<D>(qx0[j], qx1[j], qw0, qw1, a.eps, rc, rs);
        if (in_pair) {
          q_s[h][d0] = qx0[j] * qscale;
          q_s[h][d1] = qx1[j] * qscale;
        }
      }
    }
    // The new token sits in tile p / TT; only the block owning that tile
    // appends it, from its last wave, which also places the token's row in
    // that tile's LDS stage.  k and v are rounded to the cache dtype once, so
    // this step and later steps see the same key/value.
    const bool owns_new = (MODE == kAttnFused) && ((p / TT) % S == split);
    if (owns_new && wave == kAttnWaves - 1) {
      wave_norm_rope_pair<D>(kx0, kx1, kw0, kw1, a.eps, rc, rs);
      const KV k0 = from_float<KV>(kx0), k1 = from_float<KV>(kx1);
      const KV v0 = from_float<KV>(vx0), v1 = from_float<KV>(vx1);
      if (in_pair) {
        const int pp = kv_rows.page_of(p);
        KV* kdst = kv_rows.k_at(pp, p);
        KV* vdst = kv_rows.v_at(pp, p);
        kdst[d0] = k0;
        kdst[d1] = k1;
        vdst[d0] = v0;
        vdst[d1] = v1;
      }
      kx0 = to_float<KV>(k0);
      kx1 = to_float<KV>(k1);
      vx0 = to_float<KV>(v0);
      vx1 = to_float<KV>(v1);
    }

    // Fetch tile `tile`'s K/V chunks into the registers (rows clamped into
    // the context, all loads issued before any is consumed).
    auto fetch_tile = [&](int tile, int page) {
      const int t0 = tile * TT;
      const int rows = min(TT, n_keys - t0);
      const KV* ktile = kv_rows.k_at(page, t0);
      const KV* vtile = kv_rows.v_at(page, t0);
#pragma unroll
      for (int i = 0; i < kPerThread; ++i) {
        const int c = min(static_cast<int>(threadIdx.x) + i * kAttnThreads, kChunks - 1);
        const int r = min((c * CH) / D, rows - 1);
        const int64_t off = static_cast<int64_t>(r) * D + (c * CH) % D;
        kc[i] = *reinterpret_cast<const uint4*>(ktile + off);
        vc[i] = *reinterpret_cast<const uint4*>(vtile + off);
      }
    };
    // The first tile comes from the speculative registers when they hold it.
    if (!spec) fetch_tile(split, kv_rows.page_of(split * TT));
    // One tile: stage K/V, scores + online softmax, P.V; with the prefetch
    // variant, the next tile of this block is fetched meanwhile.
    auto tile_step = [&](int tile, auto prefetch) {
      const int t0 = tile * TT;
      const int rows = min(TT, n_keys - t0);
      // Page of the tile after next, for the prefetch in the next step
      // (issued now, so its latency hides behind this tile's).
      int page_after = 0;
      if constexpr (decltype(prefetch)::value) page_after = kv_rows.page_of((tile + 2 * S) * TT);
      // Rows past the context are zero-filled: P.V runs over the whole tile
      // with zero probabilities there, and 0 * (stale LDS) could be NaN.
#pragma unroll
      for (int i = 0; i < kPerThread; ++i) {
        const int c = threadIdx.x + i * kAttnThreads;
        const int r = (c * CH) / D;
        const int col = (c * CH) % D;
        if (c < kChunks && !(MODE == kAttnFused && t0 + r == p)) {
          if (r < rows) {
            chunk_to_float<KV>(kc[i], &k_s[r][col]);
            chunk_to_float<KV>(vc[i], &v_s[r][col]);
          } else {
#pragma unroll
            for (int e = 0; e < CH; ++e) {
              k_s[r][col + e] = 0.0f;
              v_s[r][col + e] = 0.0f;
            }
          }
        }
      }
      if (MODE == kAttnFused && p >= t0 && p < t0 + rows && wave == kAttnWaves - 1 && in_pair) {
        const int r = p - t0;
        k_s[r][d0] = kx0;
        k_s[r][d1] = kx1;
        v_s[r][d0] = vx0;
        v_s[r][d1] = vx1;
      }
      // The registers are free again: the next tile's loads overlap this
      // tile's scores and P.V (a compile-time choice: a guarded load would
      // make the compiler wait for it where the branches join).
      if constexpr (decltype(prefetch)::value) {
        fetch_tile(tile + S, next_page);
        next_page = page_after;
      }
      __syncthreads();

      // ---- scores and online softmax: one wave per query head ----
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int h = wave + j * kAttnWaves;
        if (h >= R) break;
        // Score in base-2 units, already divided by sqrt(d) (q is pre-scaled);
        // four independent partial sums over the dims shorten the FMA chain.
        float s = -INFINITY;
        if (lane < rows) {
          float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int dd = 0; dd < D; dd += 4) {
            const float4 kv4 = *reinterpret_cast<const float4*>(&k_s[lane][dd]);
            const float4 q4 = *reinterpret_cast<const float4*>(&q_s[h][dd]);
            dot[0] = fmaf(q4.x, kv4.x, dot[0]);
            dot[1] = fmaf(q4.y, kv4.y, dot[1]);
            dot[2] = fmaf(q4.z, kv4.z, dot[2]);
            dot[3] = fmaf(q4.w, kv4.w, dot[3]);
          }
          s = (dot[0] + dot[1]) + (dot[2] + dot[3]);
        }
        const float m_tile = group_max<kWave>(s);
        const float m_new = fmaxf(m_run[j], m_tile);
        const float alpha = m_run[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[j] - m_new);
        const float pv = lane < rows ? __builtin_amdgcn_exp2f(s - m_new) : 0.0f;
        l_run[j] = l_run[j] * alpha + group_sum<kWave>(pv);
        if (lane < TT) p_s[lane][h] = pv;
        if (lane == 0) alpha_s[h] = alpha;
        m_run[j] = m_new;
      }
      __syncthreads();

      // ---- P.V: thread = (dimension pair, token group), every head at once;
      // fixed trip count so all LDS reads of the group issue back to back ----
      if (pv_active) {
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) {
          if (h < R) {
            pacc[h].x *= alpha_s[h];
            pacc[h].y *= alpha_s[h];
          }
        }
        const int tb = pv_group * kPvTokens;
        if (R <= 4) {
#pragma unroll
          for (int i = 0; i < kPvTokens; ++i) {
            const float2 v = *reinterpret_cast<const float2*>(&v_s[tb + i][2 * pv_pair]);
            const float4 p0 = *reinterpret_cast<const float4*>(&p_s[tb + i][0]);
            pv_fma(pacc[0], p0.x, v);
            pv_fma(pacc[1], p0.y, v);
            pv_fma(pacc[2], p0.z, v);
            pv_fma(pacc[3], p0.w, v);
          }
        } else {
#pragma unroll
          for (int i = 0; i < kPvTokens; ++i) {
            const float2 v = *reinterpret_cast<const float2*>(&v_s[tb + i][2 * pv_pair]);
            const float4 p0 = *reinterpret_cast<const float4*>(&p_s[tb + i][0]);
            const float4 p1 = *reinterpret_cast<const float4*>(&p_s[tb + i][4]);
            pv_fma(pacc[0], p0.x, v);
            pv_fma(pacc[1], p0.y, v);
            pv_fma(pacc[2], p0.z, v);
            pv_fma(pacc[3], p0.w, v);
            pv_fma(pacc[4], p1.x, v);
            pv_fma(pacc[5], p1.y, v);
            pv_fma(pacc[6], p1.z, v);
            pv_fma(pacc[7], p1.w, v);
          }
        }
      }
      __syncthreads();
    };
    int tile = split;
    for (; tile + S < n_tiles; tile += S) tile_step(tile, std::true_type{});
    if (tile < n_tiles) tile_step(tile, std::false_type{});
  }

  // ---- partial (m, l, o[d]) per head; neutral when the split had no tile ----
  // The token groups' P.V sums meet in LDS (k_s is free after the last tile).
  float* red = &k_s[0][0];  // [kPvGroups][kAttnMaxGroup][D]
  if (pv_active) {
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h)
      if (h < R) *reinterpret_cast<float2*>(&red[(pv_group * kAttnMaxGroup + h) * D + 2 * pv_pair]) = pacc[h];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int h = wave + j * kAttnWaves;
    if (h < R && lane == 0) {
      float* dst = part + attn_ml_offset(g, split, h, S, R, D, a.hkv);
      dst[0] = m_run[j] * 0.6931471805599453f;  // base-2 units -> natural log (ln 2)
      dst[1] = l_run[j];
    }
  }
  __syncthreads();
  // The R heads' o rows of this (group, split) are contiguous: coalesced.
  float* obase = part + attn_o_offset(g, split, 0, S, R, D);
  for (int idx = threadIdx.x; idx < R * D; idx += kAttnThreads) {
    const int h = idx / D, dim = idx - (idx / D) * D;
    float o = 0.0f;
#pragma unroll
    for (int gidx = 0; gidx < kPvGroups; ++gidx) o += red[(gidx * kAttnMaxGroup + h) * D + dim];
    obase[idx] = o;
  }
}

// attention_mfma_kernel: attention_split_kernel's work (same grid, fused
// prologue, KV append and split partials) with the scores and P.V on the fp16
// matrix cores, for an fp16 cache and 64-token tiles (d = 32, 64, 96).  Wave w
// of the block takes keys [16 w, 16 w + 16) of each of the block's tiles: it
// stages them in its own LDS region as loaded (fp16, no conversion), so the
// waves never wait for each other inside the tile loop, and keeps its own
// online softmax; the waves merge at the end.  Per 16-key sub-tile:
//  * S^T = K Q^T on v_mfma_f32_16x16x32_f16 with q split into fp16 hi + lo
//    (two products): lane l holds S^T[key 4 (l / 16) + i][query l % 16], the
//    queries being the group's R heads (columns past R hold zero q and are
//    never written out);
//  * O^T += V^T P^T on v_mfma_f32_16x16x16f16 with p split hi + lo: the lane
//    already holds the P^T entries the B operand needs, and the V^T fragments
//    come from one transposing LDS read (ds_read_b64_tr_b16) each.
// The hi + lo splits make each product as exact as the fp32 path's; only the
// order of the fp32 sums differs.  The split kernel stages every tile as fp32
// and reads K once per head: the LDS traffic, not HBM, set its time on long
// contexts.
using f32x4 = float __attribute__((ext_vector_type(4)));
using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using f16x4 = _Float16 __attribute__((ext_vector_type(4)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using i16x4 = short __attribute__((ext_vector_type(4)));
constexpr int kMfmaKeys = 16;  // keys per wave sub-tile: one matrix-core row block

template <int D>
constexpr bool attn_mfma_supported() {
  return D % 32 == 0 && attn_tile_tokens<D>() == kAttnWaves * kMfmaKeys;
}

template <int D, int MODE, bool PAGED, int QP = 1>
__global__ __launch_bounds__(kAttnThreads) void attention_mfma_kernel(AttnArgs a) {
  using KV = __half;
  constexpr int TT = attn_tile_tokens<D>();
  static_assert(attn_mfma_supported<D>(), "one 16-key sub-tile per wave, 32-dim slices");
  constexpr int CH = 8;  // halves per 16-byte chunk
  constexpr int kRowChunks = D / CH;
  constexpr int kChunks = kMfmaKeys * kRowChunks;  // chunks of a K (or V) sub-tile
  constexpr int kPer = (kChunks + kWave - 1) / kWave;
  constexpr int LDH = D + 8;  // fp16 stage row: 16-byte aligned, rows start on shifted banks
  constexpr int DT = D / 16;  // 16-dimension output slices
  __shared__ __align__(16) float q_s[kAttnMaxGroup][D];
  __shared__ __align__(16) _Float16 stage[kAttnWaves][2][kMfmaKeys][LDH];
  __shared__ __align__(16) _Float16 new_s[2][D];  // the new token's k and v, as appended
  __shared__ float red_m[kAttnWaves][kAttnMaxGroup], red_l[kAttnWaves][kAttnMaxGroup];
  __shared__ __align__(16) float red_o[kAttnWaves][kAttnMaxGroup][D];
  static_assert(D / 2 <= kWave, "a wave holds one head as d/2 RoPE pairs");

  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int b = blockIdx.z;  // sequence of a batch (0 for a single sequence)
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int qi = lane % 16, kq = lane / 16;  // MFMA column (query head) and k slot
  const int R = a.hq / a.hkv;
  const int S = a.splits;
  const KvRows<KV, D, PAGED> kv_rows(a, b, g);
  float* part = a.part + static_cast<int64_t>(b) * a.part_stride;
  const float* qkv_row = a.qkv + static_cast<int64_t>(b) * a.qkv_stride;

  // ---- 1. independent loads, issued before the position is known: the raw
  // q/k/v (every QKV partial), gains and RoPE frequencies first, then the
  // wave's sub-tile of the block's first tile.  Vector loads complete in
  // issue order, so the q/k norm and RoPE wait for the first group alone
  // while the K/V tile is still arriving (the partials are summed after the
  // tile's loads are out) ----
  int p = -1;
  if constexpr (MODE == kAttnFused) p = ((const __attribute__((address_space(4))) int32_t*)a.pos)[b];
  const int d0 = min(lane, D / 2 - 1), d1 = d0 + D / 2;
  const bool in_pair = lane < D / 2;
  constexpr int kParts = PAGED ? QP : 1;  // QKV partials loaded, as in attention_split_kernel
  float rq0[kParts][2], rq1[kParts][2], rk0[kParts], rk1[kParts], rv0[kParts], rv1[kParts];
#pragma unroll
  for (int pt = 0; pt < kParts; ++pt) {
    const float* row = qkv_row + static_cast<int64_t>(min(pt, a.qkv_parts - 1)) * a.qkv_part_stride;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int h = min(wave + j * kAttnWaves, R - 1);
      const float* src = (MODE == kAttnFused ? row : a.q) + (g * R + h) * D;
      rq0[pt][j] = src[d0];
      rq1[pt][j] = src[d1];
    }
    rk0[pt] = rk1[pt] = rv0[pt] = rv1[pt] = 0.0f;
    if constexpr (MODE == kAttnFused) {
      const float* kraw = row + a.hq * D + g * D;
      const float* vraw = kraw + a.hkv * D;
      rk0[pt] = kraw[d0];
      rv0[pt] = vraw[d0];
      rk1[pt] = kraw[d1];
      rv1[pt] = vraw[d1];
    }
  }
  float inv_freq = 0.0f, qw0 = 0.0f, qw1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f;
  if constexpr (MODE == kAttnFused) {
    inv_freq = a.inv_freq[d0];
    qw0 = a.q_norm[d0];
    qw1 = a.q_norm[d1];
    kw0 = a.k_norm[d0];
    kw1 = a.k_norm[d1];
  }
  asm volatile("" ::: "memory");  // the loads above go out before the tile's
  uint4 kc[kPer], vc[kPer];
  const int t_spec = split * TT;
  const bool spec = t_spec + TT <= a.rows;
  const KV* kspec;
  const KV* vspec;
  kv_rows.first_tile(t_spec, spec, kspec, vspec);  // a tile is one page's contiguous rows
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = min(lane + i * kWave, kChunks - 1);
    const int off = (kMfmaKeys * wave + c / kRowChunks) * D + (c % kRowChunks) * CH;
    kc[i] = *reinterpret_cast<const uint4*>(kspec + off);
    vc[i] = *reinterpret_cast<const uint4*>(vspec + off);
  }
  int next_page = kv_rows.page_of((split + S) * TT);
  asm volatile("" ::: "memory");
  // The partials summed in order (parts past qkv_parts weighted 0).
  float qx0[2] = {0.0f, 0.0f}, qx1[2] = {0.0f, 0.0f};
  float kx0 = 0.0f, kx1 = 0.0f, vx0 = 0.0f, vx1 = 0.0f;
#pragma unroll
  for (int pt = 0; pt < kParts; ++pt) {
    const float wgt = pt < a.qkv_parts ? 1.0f : 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      qx0[j] += wgt * rq0[pt][j];
      qx1[j] += wgt * rq1[pt][j];
    }
    kx0 += wgt * rk0[pt];
    vx0 += wgt * rv0[pt];
    kx1 += wgt * rk1[pt];
    vx1 += wgt * rv1[pt];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    qx0[j] = in_pair ? qx0[j] : 0.0f;
    qx1[j] = in_pair ? qx1[j] : 0.0f;
  }
  kx0 = in_pair ? kx0 : 0.0f;
  vx0 = in_pair ? vx0 : 0.0f;
  kx1 = in_pair ? kx1 : 0.0f;
  vx1 = in_pair ? vx1 : 0.0f;

  // ---- 2. extent of the context ----
  int n_keys;
  if constexpr (MODE == kAttnFused) {
    const bool ok = p >= 0 && p < a.capacity;
    if (!ok && threadIdx.x == 0 && split == 0 && g == 0) *a.err = 1;  // vector store, once per sequence
    n_keys = ok ? p + 1 : 0;
  } else {
    n_keys = a.tokens < a.capacity ? a.tokens : a.capacity;
  }
  const int n_tiles = (n_keys + TT - 1) / TT;

  float m_run = -INFINITY, l_part = 0.0f;  // column qi's running max (base 2) and the lane's share of its sum
  f32x4 ot[DT];                            // O^T[dim 16 j + 4 kq + i][head qi]
#pragma unroll
  for (int j = 0; j < DT; ++j) ot[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  if (split < n_tiles) {
    // ---- 3. q (a wave per head) into LDS, scaled by log2(e) / sqrt(d) (the
    // scores come out divided by sqrt(d), decoder_layer.cpp:213, in base-2
    // units for exp2); the block owning the new token's tile normalises and
    // rotates its k, rounds k and v to fp16 and appends them to the cache ----
    float rc = 1.0f, rs = 0.0f;
    if constexpr (MODE == kAttnFused) {
      if (in_pair) sincosf(static_cast<float>(p) * inv_freq, &rs, &rc);
    }
    const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(D));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int h = wave + j * kAttnWaves;
      if (h < R) {
        if constexpr (MODE == kAttnFused) wave_norm_rope_pair<D>(qx0[j], qx1[j], qw0, qw1, a.eps, rc, rs);
        if (in_pair) {
          q_s[h][d0] = qx0[j] * qscale;
          q_s[h][d1] = qx1[j] * qscale;
        }
      }
    }
    const bool owns_new = (MODE == kAttnFused) && ((p / TT) % S == split);
    if (owns_new && wave == kAttnWaves - 1) {
      wave_norm_rope_pair<D>(kx0, kx1, kw0, kw1, a.eps, rc, rs);
      const KV k0 = from_float<KV>(kx0), k1 = from_float<KV>(kx1);
      const KV v0 = from_float<KV>(vx0), v1 = from_float<KV>(vx1);
      if (in_pair) {
        const int pp = kv_rows.page_of(p);
        KV* kdst = kv_rows.k_at(pp, p);
        KV* vdst = kv_rows.v_at(pp, p);
        kdst[d0] = k0;
        kdst[d1] = k1;
        vdst[d0] = v0;
        vdst[d1] = v1;
        new_s[0][d0] = __builtin_bit_cast(_Float16, k0);
        new_s[0][d1] = __builtin_bit_cast(_Float16, k1);
        new_s[1][d0] = __builtin_bit_cast(_Float16, v0);
        new_s[1][d1] = __builtin_bit_cast(_Float16, v1);
      }
    }
    __syncthreads();  // q_s and new_s

    // Q^T fragments (B operand): lane (qi, kq) holds dims 32 j + 8 kq .. + 7
    // of head qi, split into fp16 hi + lo; zero for columns past R.
    uint4 qh[D / 32], ql[D / 32];
    {
      const float* qrow = q_s[min(qi, R - 1)];
      const float use = qi < R ? 1.0f : 0.0f;
#pragma unroll
      for (int j = 0; j < D / 32; ++j) {
        const float4 x0 = *reinterpret_cast<const float4*>(qrow + 32 * j + 8 * kq);
        const float4 x1 = *reinterpret_cast<const float4*>(qrow + 32 * j + 8 * kq + 4);
        const float x[8] = {x0.x * use, x0.y * use, x0.z * use, x0.w * use,
                            x1.x * use, x1.y * use, x1.z * use, x1.w * use};
        f16x8 hv, lv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hv[e] = static_cast<_Float16>(x[e]);
          lv[e] = static_cast<_Float16>(x[e] - static_cast<float>(hv[e]));
        }
        qh[j] = __builtin_bit_cast(uint4, hv);
        ql[j] = __builtin_bit_cast(uint4, lv);
      }
    }

    _Float16* kh = &stage[wave][0][0][0];
    _Float16* vh = &stage[wave][1][0][0];
    // The wave's 16 keys of tile `tile` into the registers (rows clamped into
    // the context: keys past it are masked below).
    auto fetch = [&](int tile, int page) {
      const int t0 = tile * TT;
      const int rows = min(TT, n_keys - t0);
      const KV* ktile = kv_rows.k_at(page, t0);
      const KV* vtile = kv_rows.v_at(page, t0);
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int c = min(lane + i * kWave, kChunks - 1);
        const int r = min(kMfmaKeys * wave + c / kRowChunks, rows - 1);
        const int64_t off = static_cast<int64_t>(r) * D + (c % kRowChunks) * CH;
        kc[i] = *reinterpret_cast<const uint4*>(ktile + off);
        vc[i] = *reinterpret_cast<const uint4*>(vtile + off);
      }
    };
    if (!spec) fetch(split, kv_rows.page_of(split * TT));

    auto step = [&](int tile, auto prefetch) {
      const int key0 = tile * TT + kMfmaKeys * wave;
      int page_after = 0;
      if constexpr (decltype(prefetch)::value) page_after = kv_rows.page_of((tile + 2 * S) * TT);
      // Stage the sub-tile as loaded, rows past the context as zeros (the
      // speculative first tile reads whole pages, whose unwritten rows may
      // hold any bits, and P.V multiplies every row: 0 * NaN is NaN); the new
      // token's row from new_s instead of the cache (written by this launch).
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int c = lane + i * kWave;
        if (c < kChunks) {
          const int r = c / kRowChunks, col = (c % kRowChunks) * CH;
          const uint32_t keep = key0 + r < n_keys ? ~0u : 0u;
          const uint4 k4 = kc[i], v4 = vc[i];
          *reinterpret_cast<u32x4*>(&kh[r * LDH + col]) = u32x4{k4.x & keep, k4.y & keep, k4.z & keep, k4.w & keep};
          *reinterpret_cast<u32x4*>(&vh[r * LDH + col]) = u32x4{v4.x & keep, v4.y & keep, v4.z & keep, v4.w & keep};
        }
      }
      if (MODE == kAttnFused && p >= key0 && p < key0 + kMfmaKeys && lane < kRowChunks) {
        const int r = p - key0;
        *reinterpret_cast<uint4*>(&kh[r * LDH + lane * CH]) = *reinterpret_cast<const uint4*>(&new_s[0][lane * CH]);
        *reinterpret_cast<uint4*>(&vh[r * LDH + lane * CH]) = *reinterpret_cast<const uint4*>(&new_s[1][lane * CH]);
      }
      // The registers are free: the next tile's loads overlap this one's work
      // (a compile-time choice; a guarded load would be waited for where the
      // branches join).
      if constexpr (decltype(prefetch)::value) {
        fetch(tile + S, next_page);
        next_page = page_after;
      }
      // The stage is the wave's own and its LDS operations complete in order:
      // waiting for the writes suffices before other lanes read them.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < D / 32; ++j) {
        const f16x8 kf = *reinterpret_cast<const f16x8*>(&kh[qi * LDH + 32 * j + 8 * kq]);
        st = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(f16x8, qh[j]), st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(f16x8, ql[j]), st, 0, 0, 0);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st[i] = key0 + 4 * kq + i < n_keys ? st[i] : -INFINITY;
        mx = fmaxf(mx, st[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      // No key of this column seen yet (m_new = -inf): everything stays zero.
      const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_part *= alpha;
#pragma unroll
      for (int j = 0; j < DT; ++j) ot[j] *= alpha;
      f16x4 ph, pl;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = st[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st[i] - m_new);
        l_part += pv;
        ph[i] = static_cast<_Float16>(pv);
        pl[i] = static_cast<_Float16>(pv - static_cast<float>(ph[i]));
      }
      m_run = m_new;
#pragma unroll
      for (int j = 0; j < DT; ++j) {
        // A = V^T: lane (qi, kq) needs V[key 4 kq + i][dim 16 j + qi], i =
        // 0..3; the transposing read gives lane i of a 16-lane group element
        // i % 4 of the 8 bytes lane 4 k + i / 4 addresses (k = 0..3), so lane
        // qi addresses key 4 kq + qi / 4, dims 16 j + 4 (qi % 4) .. + 3.
        const _Float16* vsrc = &vh[(4 * kq + qi / 4) * LDH + 16 * j + 4 * (qi % 4)];
        const f16x4 va = __builtin_bit_cast(
            f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(vsrc)));
        ot[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, ot[j], 0, 0, 0);
        ot[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, ot[j], 0, 0, 0);
      }
      // Reads of this stage finish before the next tile's writes (in-order LDS).
    };
    // Blocks with one tile (every block while the splits cover the tiles, as
    // in single-sequence steps) take a path of their own, without the loop:
    // MiniMind2 decode at 8,192 keys 369.4 -> 364.6 us per step, batched
    // step p50 0.774 -> 0.770 ms (same box, two runs each).
    int tile = split;
    if (tile + S < n_tiles) {
      for (; tile + S < n_tiles; tile += S) step(tile, std::true_type{});
      step(tile, std::false_type{});
    } else {
      step(tile, std::false_type{});
    }
  }

  // ---- 4. merge the waves: per head, M = max of the waves' m, then
  // o = sum_w e_w o_w and l = sum_w e_w l_w with e_w = exp2(m_w - M), in wave
  // order; neutral (-inf, 0, 0) when the split had no tile ----
  float l = l_part + __shfl_xor(l_part, 16);
  l += __shfl_xor(l, 32);
  if (qi < R) {
    if (kq == 0) {
      red_m[wave][qi] = m_run;
      red_l[wave][qi] = l;
    }
#pragma unroll
    for (int j = 0; j < DT; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) red_o[wave][qi][16 * j + 4 * kq + i] = ot[j][i];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * D; idx += kAttnThreads) {
    const int h = idx / D, dim = idx - (idx / D) * D;
    float M = red_m[0][h];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, red_m[w][h]);
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w)
      o = fmaf(M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w][h] - M), red_o[w][h][dim], o);
    part[attn_o_offset(g, split, 0, S, R, D) + idx] = o;
  }
  if (static_cast<int>(threadIdx.x) < R) {
    const int h = threadIdx.x;
    float M = red_m[0][h];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, red_m[w][h]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w)
      L = fmaf(M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w][h] - M), red_l[w][h], L);
    float* dst = part + attn_ml_offset(g, split, h, S, R, D, a.hkv);
    dst[0] = M * 0.6931471805599453f;  // base-2 units -> natural log (ln 2)
    dst[1] = L;
  }
}

// attention_head_kernel, splits * hq blocks of kHW = head_kernel_waves()
// waves (512 threads for d 32-128): the contiguous-cache (single-sequence)
// variant.  Block (s, h) serves query head h of KV group g = h / R over the
// tiles s, s + splits, ...  The R blocks of a group stage the same K/V tile:
// a single-sequence step has few tiles, and four times the blocks spreads the
// scores and P.V over four times the CUs.  Inside the block, wave w owns
// tokens [w, w + 1) * TT / kHW of each tile with its own online softmax; the
// waves' (m, l, o) merge at the end.
//  * scores: the kLanesPerTok adjacent lanes of a token each sum an
//    interleaved share of the dims (16-byte columns c * kLanesPerTok + share),
//    then add across the share with DPP;
//  * P.V: one lane per dimension pair over the wave's tokens, the
//    probabilities read out of the scoring lanes.
// Writes the same (m, l, o[d]) split partials as attention_split_kernel.
// kHeads = 4 (four waves per head, 1024 threads, one block per (split,
// group)): the group's four heads share one staged tile, waves 4 j .. 4 j + 3
// serving head j as a one-head block of four waves would; the long-context
// form, one staging per tile instead of four while keeping a short chain.
template <typename KV, int D, int MODE, int kHeads>
__global__ __launch_bounds__((head_kernel_waves<D, kHeads>() * kWave * kHeads)) void attention_head_kernel(AttnArgs a) {
  constexpr int TT = attn_tile_tokens<D>();
  constexpr int LD = D + 4;
  constexpr int CH = 16 / static_cast<int>(sizeof(KV));
  constexpr int kChunks = TT * D / CH;
  constexpr int kHW = head_kernel_waves<D, kHeads>();  // waves per head
  constexpr int kThreads = kHW * kWave * kHeads;
  constexpr int kWaves = kThreads / kWave;
  constexpr int kPerThread = (kChunks + kThreads - 1) / kThreads;
  constexpr int kPairs = D / 2;
  constexpr int kTokPerWave = TT / kHW;
  constexpr int kLanesPerTok = kWave / kTokPerWave;
  constexpr int kQuadsPerLane = D / 4 / kLanesPerTok;
  static_assert(TT % kHW == 0 && kWave % kTokPerWave == 0, "a wave holds whole tokens");
  static_assert((D / 4) % kLanesPerTok == 0, "the dims split evenly over a token's lanes");
  static_assert(D / 2 <= kWave, "a wave holds one head as d/2 RoPE pairs");
  __shared__ __align__(16) float q_s[kHeads][D];
  __shared__ __align__(16) float k_s[TT][LD];
  __shared__ __align__(16) float v_s[TT][LD];
  __shared__ __align__(16) float red_o[kWaves][D];
  __shared__ float red_m[kWaves], red_l[kWaves];

  const int R = a.hq / a.hkv;
  const int S = a.splits;
  // Blocks past the S * hq head blocks: padding up to a multiple of kXcds,
  // then the L2-warming blocks (their loads land in k_s, which they own).
  static_assert(kHeads > 1 || sizeof(k_s) >= kWaves * kWave * 16, "a 1 KB landing zone per wave");
  if constexpr (kHeads == 1) {
    if (static_cast<int>(blockIdx.x) >= S * a.hq) {
      const int first = (S * a.hq + kXcds - 1) / kXcds * kXcds;
      if (MODE == kAttnFused && static_cast<int>(blockIdx.x) >= first)
        l2_warm<kThreads>(a.warm, static_cast<int>(blockIdx.x) - first, &k_s[0][0]);
      return;
    }
  }
  // Block -> (split, group, head): the R head-blocks of one (split, group)
  // unit take ids 8 apart, so the round-robin dispatch over the 8 XCDs puts
  // them on one XCD and their K/V tile is read from HBM into one L2.  (A
  // last partial group of 8 units keeps its blocks together less tightly.)
  // With kHeads = R, block (split, group) is one unit and its four waves
  // 4 j .. 4 j + 3 serve head j of the group from the one staged tile.
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int wq = kHeads == 1 ? wave : wave % kHW;  // the wave's token group of the tile
  const int hb = kHeads == 1 ? 0 : wave / kHW;     // the wave's head within the block
  int unit, r;
  if constexpr (kHeads == 1) {
    const int units = S * a.hkv;
    const int full = units / 8 * 8;
    const int id = blockIdx.x;
    if (id < full * R) {
      const int w = id % (8 * R);
      unit = id / (8 * R) * 8 + w % 8;
      r = w / 8;
    } else {
      const int tail = units - full, w = id - full * R;
      unit = full + w % tail;
      r = w / tail;
    }
  } else {
    unit = blockIdx.x;
    r = hb;
  }
  const int split = unit / a.hkv;
  const int g = unit % a.hkv;
  const int h = g * R + r;
  const KvRows<KV, D, false> kv_rows(a, 0, g);

  // ---- 1. independent loads, issued before the position is known ----
  // The position is read through the scalar cache (no kernel writes it while
  // this one runs): its wait (lgkmcnt) never covers the vector loads below,
  // which go out at once instead of behind one memory round trip.
  int p = -1;
  if constexpr (MODE == kAttnFused) p = *(const __attribute__((address_space(4))) int32_t*)a.pos;
  // The new token's q / k / v, the norm gains and the RoPE frequencies come
  // first: vector loads complete in issue order, so the q norm and RoPE wait
  // for these alone while the K/V tile below is still arriving.
  // Lane i < d/2 holds dims (i, i + d/2), the pair RoPE rotates together.
  // Every lane loads (d0 is clamped, so in bounds): a guarded load is a
  // branch, and the compiler waits for its data where the branches join.
  // Lanes past d/2 are zeroed once the K/V tile loads are out.
  const int d0 = min(lane, D / 2 - 1), d1 = d0 + D / 2;
  const bool in_pair = lane < D / 2;
  const float* qsrc = (MODE == kAttnFused ? a.qkv : a.q) + h * D;
  float qx0 = qsrc[d0], qx1 = qsrc[d1];
  float kx0 = 0.0f, kx1 = 0.0f, vx0 = 0.0f, vx1 = 0.0f, inv_freq = 0.0f;
  float qw0 = 0.0f, qw1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f;
  if constexpr (MODE == kAttnFused) {
    const float* kraw = a.qkv + a.hq * D + g * D;
    const float* vraw = kraw + a.hkv * D;
    kx0 = kraw[d0];
    kx1 = kraw[d1];
    vx0 = vraw[d0];
    vx1 = vraw[d1];
    inv_freq = a.inv_freq[d0];
    qw0 = a.q_norm[d0];
    qw1 = a.q_norm[d1];
    kw0 = a.k_norm[d0];
    kw1 = a.k_norm[d1];
  }
  uint4 kc[kPerThread], vc[kPerThread];
  const int t_spec = split * TT;
  const bool spec = t_spec + TT <= a.rows;
  const KV* kspec;
  const KV* vspec;
  kv_rows.first_tile(t_spec, spec, kspec, vspec);  // always backed; unused unless spec
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int c = min(static_cast<int>(threadIdx.x) + i * kThreads, kChunks - 1);
    kc[i] = *reinterpret_cast<const uint4*>(kspec + c * CH);
    vc[i] = *reinterpret_cast<const uint4*>(vspec + c * CH);
  }
  asm volatile("" ::: "memory");
  if (!in_pair) qx0 = qx1 = kx0 = kx1 = vx0 = vx1 = 0.0f;

  // ---- 2. extent of the context ----
  int n_keys;
  if constexpr (MODE == kAttnFused) {
    const bool ok = p >= 0 && p < a.capacity;
    if (!ok && threadIdx.x == 0 && split == 0 && h == 0) *a.err = 1;  // vector store, once
    n_keys = ok ? p + 1 : 0;
  } else {
    n_keys = a.tokens < a.capacity ? a.tokens : a.capacity;
  }
  const int n_tiles = (n_keys + TT - 1) / TT;

  // The wave's running softmax state and P.V sums (lane i < d/2: dims 2i, 2i + 1).
  float m_run = -INFINITY, l_run = 0.0f;
  float2 pacc = make_float2(0.0f, 0.0f);
  const int pv_pair = min(lane, kPairs - 1);
  const int tok = wq * kTokPerWave + lane / kLanesPerTok;  // scoring token within the tile
  const int share = lane % kLanesPerTok;  // which interleaved share of the dims
  bool append_new = false;  // this lane writes dims (d0, d1) of cache row p at the end

  if (split < n_tiles) {
    // ---- 3. q (wave 0) and the new key/value (wave 1), in registers ----
    float rc = 1.0f, rs = 0.0f;
    if constexpr (MODE == kAttnFused) {
      if (in_pair) sincosf(static_cast<float>(p) * inv_freq, &rs, &rc);
    }
    if (wq == 0) {  // one wave per head
      if constexpr (MODE == kAttnFused) wave_norm_rope_pair<D>(qx0, qx1, qw0, qw1, a.eps, rc, rs);
      // q staged times log2(e) / sqrt(d): the scores come out divided by
      // sqrt(d) (decoder_layer.cpp:213) and in base-2 units for exp2.
      const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(D));
      if (in_pair) {
        q_s[hb][d0] = qx0 * qscale;
        q_s[hb][d1] = qx1 * qscale;
      }
    }
    // The block owning tile p / TT places the new token's row in its stage;
    // the first block of the group also appends it to the cache.  k and v
    // are rounded to the cache dtype once, so this step and later steps see
    // the same key/value.
    const bool owns_new = (MODE == kAttnFused) && ((p / TT) % S == split);
    if (owns_new && wave == 1) {
      wave_norm_rope_pair<D>(kx0, kx1, kw0, kw1, a.eps, rc, rs);
      kx0 = to_float<KV>(from_float<KV>(kx0));
      kx1 = to_float<KV>(from_float<KV>(kx1));
      vx0 = to_float<KV>(from_float<KV>(vx0));
      vx1 = to_float<KV>(from_float<KV>(vx1));
      // The cache row is written at the end of the kernel: this block takes
      // the new row from registers, the other blocks of the launch never read
      // row p from the cache, and a store issued here would be waited for by
      // the vector-memory waits of the staging below.
      append_new = in_pair && r == 0;
    }

    auto fetch_tile = [&](int tile) {
      const int t0 = tile * TT;
      const int rows = min(TT, n_keys - t0);
      const int seg = kv_rows.page_of(t0);
      const KV* ktile = kv_rows.k_at(seg, t0);
      const KV* vtile = kv_rows.v_at(seg, t0);
#pragma unroll
      for (int i = 0; i < kPerThread; ++i) {
        const int c = min(static_cast<int>(threadIdx.x) + i * kThreads, kChunks - 1);
        const int r = min((c * CH) / D, rows - 1);
        const int64_t off = static_cast<int64_t>(r) * D + (c * CH) % D;
        kc[i] = *reinterpret_cast<const uint4*>(ktile + off);
        vc[i] = *reinterpret_cast<const uint4*>(vtile + off);
      }
    };
    if (!spec) fetch_tile(split);
    auto tile_step = [&](int tile, auto prefetch) {
      const int t0 = tile * TT;
      const int rows = min(TT, n_keys - t0);
      // Rows past the context are zero-filled (0 * stale LDS could be NaN).
#pragma unroll
      for (int i = 0; i < kPerThread; ++i) {
        const int c = threadIdx.x + i * kThreads;
        const int r = (c * CH) / D;
        const int col = (c * CH) % D;
        if (c < kChunks && !(MODE == kAttnFused && t0 + r == p)) {
          if (r < rows) {
            chunk_to_float<KV>(kc[i], &k_s[r][col]);
            chunk_to_float<KV>(vc[i], &v_s[r][col]);
          } else {
#pragma unroll
            for (int e = 0; e < CH; ++e) {
              k_s[r][col + e] = 0.0f;
              v_s[r][col + e] = 0.0f;
            }
          }
        }
      }
      if (MODE == kAttnFused && p >= t0 && p < t0 + rows && wave == 1 && in_pair) {
        const int r = p - t0;
        k_s[r][d0] = kx0;
        k_s[r][d1] = kx1;
        v_s[r][d0] = vx0;
        v_s[r][d1] = vx1;
      }
      if constexpr (decltype(prefetch)::value) fetch_tile(tile + S);
      __syncthreads();

      // Every LDS read of the tile step goes out before any arithmetic: the
      // K and q shares for the scores, then the wave's V rows for P.V.  LDS
      // returns in order, so the scores wait for K and q alone and the V rows
      // arrive while the softmax runs (left to itself the compiler keeps two
      // V reads in flight and waits on each).
      float4 k4[kQuadsPerLane], q4[kQuadsPerLane];
#pragma unroll
      for (int c = 0; c < kQuadsPerLane; ++c) {
        const int col = 4 * (c * kLanesPerTok + share);
        k4[c] = *reinterpret_cast<const float4*>(&k_s[tok][col]);
        q4[c] = *reinterpret_cast<const float4*>(&q_s[hb][col]);
      }
      float2 vrow[kTokPerWave];
#pragma unroll
      for (int t = 0; t < kTokPerWave; ++t)
        vrow[t] = *reinterpret_cast<const float2*>(&v_s[wq * kTokPerWave + t][2 * pv_pair]);
      asm volatile("" : : : "memory");

      // ---- scores of the wave's tokens ----
      float dot = 0.0f;
#pragma unroll
      for (int c = 0; c < kQuadsPerLane; ++c) {
        dot = fmaf(q4[c].x, k4[c].x, dot);
        dot = fmaf(q4[c].y, k4[c].y, dot);
        dot = fmaf(q4[c].z, k4[c].z, dot);
        dot = fmaf(q4[c].w, k4[c].w, dot);
      }
      dot = group_sum<kLanesPerTok>(dot);
      const bool live = tok < rows;
      const float sc = live ? dot : -INFINITY;  // score / sqrt(d), times log2(e)
      // ---- the wave's online softmax in base 2 (a wave may have no live
      // token yet) ----
      const float m_new = fmaxf(m_run, group_max<kWave>(sc));
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float pv = live ? __builtin_amdgcn_exp2f(sc - m_new) : 0.0f;
      l_run = l_run * alpha + group_sum<kWave>(share == 0 ? pv : 0.0f);
      m_run = m_new;
      // ---- P.V over the wave's tokens ----
      float2 acc = make_float2(pacc.x * alpha, pacc.y * alpha);
#pragma unroll
      for (int t = 0; t < kTokPerWave; ++t) {
        const float pt = lane_value(pv, t * kLanesPerTok);
        acc.x = fmaf(pt, vrow[t].x, acc.x);
        acc.y = fmaf(pt, vrow[t].y, acc.y);
      }
      pacc = acc;
      // The next tile's staging overwrites k_s / v_s: every wave must be done.
      if constexpr (decltype(prefetch)::value) __syncthreads();
    };
    int tile = split;
    for (; tile + S < n_tiles; tile += S) tile_step(tile, std::true_type{});
    if (tile < n_tiles) tile_step(tile, std::false_type{});
  }

  // ---- merge the waves' (m, l, o) in wave order; neutral when the split had
  // no tile.  m is in base-2 units until the store, which converts it to the
  // natural-log units of the split partials. ----
  if (lane < kPairs) *reinterpret_cast<float2*>(&red_o[wave][2 * lane]) = pacc;
  if (lane == 0) {
    red_m[wave] = m_run;
    red_l[wave] = l_run;
  }
  __syncthreads();
  if constexpr (kHeads == 1) {
    float M = red_m[0];
#pragma unroll
    for (int w = 1; w < kHW; ++w) M = fmaxf(M, red_m[w]);
    float e[kHW];
#pragma unroll
    for (int w = 0; w < kHW; ++w) e[w] = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w] - M);
    for (int idx = threadIdx.x; idx < D; idx += kThreads) {
      float o = 0.0f;
#pragma unroll
      for (int w = 0; w < kHW; ++w) o = fmaf(e[w], red_o[w][idx], o);
      a.part[attn_o_offset(g, split, r, S, R, D) + idx] = o;
    }
    if (threadIdx.x == 0) {
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < kHW; ++w) L = fmaf(e[w], red_l[w], L);
      float* dst = a.part + attn_ml_offset(g, split, r, S, R, D, a.hkv);
      dst[0] = M * 0.6931471805599453f;  // ln 2
      dst[1] = L;
    }
  } else {
    // Head j of the block: waves 4 j .. 4 j + 3.
    for (int idx = threadIdx.x; idx < kHeads * D; idx += kThreads) {
      const int j = idx / D, dim = idx - j * D;
      float M = red_m[kHW * j];
  #pragma unroll
      for (int w = 1; w < kHW; ++w) M = fmaxf(M, red_m[kHW * j + w]);
      float o = 0.0f;
  #pragma unroll
      for (int w = 0; w < kHW; ++w) {
        const float e = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[kHW * j + w] - M);
        o = fmaf(e, red_o[kHW * j + w][dim], o);
      }
      a.part[attn_o_offset(g, split, r - hb + j, S, R, D) + dim] = o;
    }
    if (static_cast<int>(threadIdx.x) < kHeads) {
      const int j = threadIdx.x;
      float M = red_m[kHW * j];
  #pragma unroll
      for (int w = 1; w < kHW; ++w) M = fmaxf(M, red_m[kHW * j + w]);
      float L = 0.0f;
  #pragma unroll
      for (int w = 0; w < kHW; ++w)
        L = fmaf(M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[kHW * j + w] - M), red_l[kHW * j + w], L);
      float* dst = a.part + attn_ml_offset(g, split, r - hb + j, S, R, D, a.hkv);
      dst[0] = M * 0.6931471805599453f;  // ln 2
      dst[1] = L;
    }
  }
  // The new token's k / v (rounded to the cache dtype above), after every
  // other memory operation of the block.
  if (append_new) {
    const int seg = kv_rows.page_of(p);
    KV* kdst = kv_rows.k_at(seg, p);
    KV* vdst = kv_rows.v_at(seg, p);
    kdst[d0] = from_float<KV>(kx0);
    kdst[d1] = from_float<KV>(kx1);
    vdst[d0] = from_float<KV>(vx0);
    vdst[d1] = from_float<KV>(vx1);
  }
}

// Log-sum-exp combine of the split partials: one block of 256 threads per
// (query head, 16-dimension slice) (grid.y: sequence of a batch); sixteen
// groups of 16 threads (thread = dimension), group j taking splits j, j + 16,
// ...  Every thread loads the o values of its splits together with their
// (m, l) pairs, so up to 16 * kRound splits cost one memory round trip: the
// block's max M = max m (wave DPP max, then LDS), then each group sums
// e_s o_s and e_s l_s with e_s = exp(m_s - M) in split order, and the groups'
// sums meet in LDS and are added in group order.  Every order is fixed, so
// the result is deterministic.  kMulti (more than 16 * kRound splits): M
// first from every split's m (thread t: splits t, t + 256, ...), then rounds
// of 16 * kRound splits.  (The O-projection prologue, kProAttnCombine,
// computes the same quantity for up to kCombineMaxSplits splits.)
constexpr int kCombineThreads = 256;
constexpr int kCombineSlice = 16;                                   // dimensions per block
constexpr int kCombineGroups = kCombineThreads / kCombineSlice;     // split groups
constexpr int kCombineKernelMaxSplits = 4096;
constexpr int kCombineMaxPerThread = kCombineKernelMaxSplits / kCombineThreads;

// Blocks past the first multiple of kXcds at or above the merge blocks (one
// sequence only) are L2-warming blocks for `warm` (see L2WarmSet).
template <int kRound, bool kMulti>
__global__ __launch_bounds__(kCombineThreads) void attention_combine_kernel(const float* part, int hq, int hkv, int d,
                                                                             int splits, int64_t part_stride,
                                                                             float* out, L2WarmSet warm) {
  __shared__ float s_red[kCombineGroups][kCombineSlice];
  __shared__ float s_l[kCombineGroups];
  __shared__ float s_m[kCombineThreads / kWave];
  __shared__ __align__(16) uint32_t s_warm[kCombineThreads / kWave][kWave * 4];  // l2_warm scratch, 1 KB per wave
  const int nslice = (d + kCombineSlice - 1) / kCombineSlice;
  if (warm.blocks > 0) {
    const int first = (hq * nslice + kXcds - 1) / kXcds * kXcds;
    if (static_cast<int>(blockIdx.x) >= first) {
      l2_warm<kCombineThreads>(warm, static_cast<int>(blockIdx.x) - first, &s_warm[0][0]);
      return;
    }
    if (static_cast<int>(blockIdx.x) >= hq * nslice) return;  // padding up to the first warming block
  }
  const int qh = blockIdx.x / nslice, slice = blockIdx.x % nslice;
  part += static_cast<int64_t>(blockIdx.y) * part_stride;  // sequence of a batch
  out += static_cast<int64_t>(blockIdx.y) * hq * d;
  const int R = hq / hkv;
  const int g = qh / R, h = qh % R;
  const int tid = threadIdx.x;
  const int grp = tid / kCombineSlice, col = tid % kCombineSlice;
  const int dim = slice * kCombineSlice + col;
  const int dd = min(dim, d - 1);
  // Loads of one round: o and (m, l) of splits base + grp + 16 u, indices
  // clamped into range (the repeats are weighted 0), all issued together.
  float v[kRound];
  float2 ml[kRound];
  auto load_round = [&](int base) {
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      const int sp = min(base + grp + kCombineGroups * u, splits - 1);
      v[u] = part[attn_o_offset(g, sp, h, splits, R, d) + dd];
      ml[u] = *reinterpret_cast<const float2*>(part + attn_ml_offset(g, sp, h, splits, R, d, hkv));
    }
  };
  float m_loc = -INFINITY;
  if constexpr (kMulti) {
    float mm[kCombineMaxPerThread];
#pragma unroll
    for (int j = 0; j < kCombineMaxPerThread; ++j)
      mm[j] = part[attn_ml_offset(g, min(tid + j * kCombineThreads, splits - 1), h, splits, R, d, hkv)];
    load_round(0);
#pragma unroll
    for (int j = 0; j < kCombineMaxPerThread; ++j) m_loc = fmaxf(m_loc, mm[j]);  // clamped repeats: max unchanged
  } else {
    load_round(0);
#pragma unroll
    for (int u = 0; u < kRound; ++u) m_loc = fmaxf(m_loc, ml[u].x);
  }
  m_loc = group_max<kWave>(m_loc);
  if (tid % kWave == 0) s_m[tid / kWave] = m_loc;
  __syncthreads();
  float M = s_m[0];
#pragma unroll
  for (int w = 1; w < kCombineThreads / kWave; ++w) M = fmaxf(M, s_m[w]);
  float o = 0.0f, l = 0.0f;
  for (int base = 0;;) {
#pragma unroll
    for (int u = 0; u < kRound; ++u) {
      // e^x as 2^(x log2 e) on v_exp_f32: a few instructions against expf's
      // range reduction, for up to 32 weights per thread.
      const float e = base + grp + kCombineGroups * u < splits
                          ? __builtin_amdgcn_exp2f((ml[u].x - M) * 1.4426950408889634f)
                          : 0.0f;
      o = fmaf(v[u], e, o);
      l = fmaf(ml[u].y, e, l);
    }
    base += kCombineGroups * kRound;
    if (!kMulti || base >= splits) break;
    load_round(base);
  }
  s_red[grp][col] = o;
  if (col == 0) s_l[grp] = l;
  __syncthreads();
  if (grp == 0 && dim < d) {
    float x = s_red[0][col], L = s_l[0];
#pragma unroll
    for (int gi = 1; gi < kCombineGroups; ++gi) {
      x += s_red[gi][col];
      L += s_l[gi];
    }
    out[qh * d + dim] = x * (1.0f / L);
  }
}

// Standalone post-process (reference K2): one wave per head, lane i < d/2
// holding the RoPE pair (i, i + d/2).
template <typename KV, int D>
__global__ __launch_bounds__(kWave) void qkv_postprocess_kernel(QkvPostArgs a) {
  static_assert(D / 2 <= kWave, "a wave holds one head as d/2 RoPE pairs");
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const bool is_q = b < a.hq;
  const int head = is_q ? b : b - a.hq;
  const float* src = a.qkv + (is_q ? head * D : a.hq * D + head * D);
  const float* w = is_q ? a.q_norm : a.k_norm;
  const bool in_pair = lane < D / 2;
  const int d0 = min(lane, D / 2 - 1), d1 = d0 + D / 2;
  float x0 = in_pair ? src[d0] : 0.0f;
  float x1 = in_pair ? src[d1] : 0.0f;
  float rc = 1.0f, rs = 0.0f;
  if (in_pair) sincosf(static_cast<float>(a.position) * a.inv_freq[d0], &rs, &rc);
  wave_norm_rope_pair<D>(x0, x1, w[d0], w[d1], a.eps, rc, rs);
  if (!in_pair) return;
  if (is_q) {
    a.query_out[head * D + d0] = x0;
    a.query_out[head * D + d1] = x1;
  } else {
    const float* vsrc = a.qkv + a.hq * D + a.hkv * D + head * D;
    const int seg = kv_segment(a.index);
    const int64_t off = kv_segment_offset(seg, a.index, head, a.hkv, D);
    KV* kdst = static_cast<KV*>(a.seg.s[seg].k) + off;
    KV* vdst = static_cast<KV*>(a.seg.s[seg].v) + off;
    kdst[d0] = from_float<KV>(x0);
    kdst[d1] = from_float<KV>(x1);
    vdst[d0] = from_float<KV>(vsrc[d0]);
    vdst[d1] = from_float<KV>(vsrc[d1]);
  }
}

// The per-head kernel re-stages each K/V tile once per query head of the
// group; past this many blocks (long contexts, many splits) one block per
// (split, group) serving every head of the group is faster.
constexpr int kHeadKernelMaxBlocks = 512;

// Query heads per KV group that the per-head kernel serves in one block
// (four waves each) past kHeadKernelMaxBlocks head blocks, while the blocks
// fit one round on the GPU (one 1024-thread block per CU): beyond, the block
// holding the newest tile could wait for a second round, and the split
// kernel (256-thread blocks, several per CU) runs.
constexpr int kGroupBlockHeads = 4;
constexpr int kGroupBlockMaxBlocks = 256;

// The split-K launch: on the fp16 matrix cores where the cache is fp16 and
// the tile is 64 keys, else the fp32 split kernel.
template <typename KV, int D, int MODE, bool PAGED, int QP = 1>
void launch_split(const AttnArgs& a, dim3 grid, hipStream_t s) {
  if constexpr (std::is_same<KV, __half>::value && attn_mfma_supported<D>()) {
    attention_mfma_kernel<D, MODE, PAGED, QP><<<grid, kAttnThreads, 0, s>>>(a);
  } else {
    attention_split_kernel<KV, D, MODE, PAGED, QP><<<grid, kAttnThreads, 0, s>>>(a);
  }
}

template <typename KV, int D>
hipError_t launch_attn_d(const AttnArgs& a, AttnMode mode, hipStream_t s) {
  const dim3 group_grid(a.splits, a.hkv, a.batch);
  if (a.page_table) {
    if (mode != kAttnFused) return hipErrorInvalidValue;
    // Each QKV partial is a load per q/k/v value in the prologue: few parts
    // take the variant that issues only kAttnFewQkvParts of them.
    if (a.qkv_parts <= kAttnFewQkvParts)
      launch_split<KV, D, kAttnFused, true, kAttnFewQkvParts>(a, group_grid, s);
    else
      launch_split<KV, D, kAttnFused, true, kAttnMaxQkvParts>(a, group_grid, s);
  } else if (static_cast<int64_t>(a.splits) * a.hq <= kHeadKernelMaxBlocks) {
    int blocks = a.splits * a.hq;
    if (mode == kAttnFused && a.warm.blocks > 0) {
      if (a.warm.blocks % kXcds != 0) return hipErrorInvalidValue;
      blocks = (blocks + kXcds - 1) / kXcds * kXcds + a.warm.blocks;
    }
    const dim3 head_grid(blocks), head_block(head_kernel_waves<D, 1>() * kWave);
    if (mode == kAttnFused) {
      attention_head_kernel<KV, D, kAttnFused, 1><<<head_grid, head_block, 0, s>>>(a);
    } else {
      attention_head_kernel<KV, D, kAttnFromCache, 1><<<head_grid, head_block, 0, s>>>(a);
    }
  } else if (!(std::is_same<KV, __half>::value && attn_mfma_supported<D>()) && a.hq / a.hkv == kGroupBlockHeads &&
             static_cast<int64_t>(a.splits) * a.hkv <= kGroupBlockMaxBlocks) {
    // Long contexts, groups of four query heads: one 1024-thread block per
    // (split, group) stages each tile once for the four heads.  (An fp16
    // cache with 64-key tiles takes the matrix-core split kernel instead:
    // MiniMind2 at 4096 keys, 326.3 against 328.1 us per step, same box.)
    const dim3 unit_grid(a.splits * a.hkv), group_block(kGroupBlockHeads * kAttnThreads);
    if (mode == kAttnFused) {
      attention_head_kernel<KV, D, kAttnFused, kGroupBlockHeads><<<unit_grid, group_block, 0, s>>>(a);
    } else {
      attention_head_kernel<KV, D, kAttnFromCache, kGroupBlockHeads><<<unit_grid, group_block, 0, s>>>(a);
    }
  } else if (mode == kAttnFused) {
    launch_split<KV, D, kAttnFused, false>(a, group_grid, s);
  } else {
    launch_split<KV, D, kAttnFromCache, false>(a, group_grid, s);
  }
  return hipGetLastError();
}

template <typename KV>
hipError_t launch_attn_kv(const AttnArgs& a, AttnMode mode, hipStream_t s) {
  switch (a.d) {
    case 16: return launch_attn_d<KV, 16>(a, mode, s);
    case 32: return launch_attn_d<KV, 32>(a, mode, s);
    case 64: return launch_attn_d<KV, 64>(a, mode, s);
    case 96: return launch_attn_d<KV, 96>(a, mode, s);
    case 128: return launch_attn_d<KV, 128>(a, mode, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename KV>
hipError_t launch_post_kv(const QkvPostArgs& a, hipStream_t s) {
  const dim3 grid(a.hq + a.hkv), block(kWave);
  switch (a.d) {
    case 16: qkv_postprocess_kernel<KV, 16><<<grid, block, 0, s>>>(a); break;
    case 32: qkv_postprocess_kernel<KV, 32><<<grid, block, 0, s>>>(a); break;
    case 64: qkv_postprocess_kernel<KV, 64><<<grid, block, 0, s>>>(a); break;
    case 96: qkv_postprocess_kernel<KV, 96><<<grid, block, 0, s>>>(a); break;
    case 128: qkv_postprocess_kernel<KV, 128><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool attention_supported(int hq, int hkv, int d) {
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0 || hq / hkv > kAttnMaxGroup) return false;
  return d == 16 || d == 32 || d == 64 || d == 96 || d == 128;
}

int attention_tile_tokens(int d) { return d <= 96 ? 64 : 32; }

size_t attention_partial_floats(int hq, int hkv, int d, int splits) {
  return static_cast<size_t>(hkv) * splits * (hq / hkv) * (d + 2);
}

hipError_t launch_attention(const AttnArgs& a, AttnMode mode, KvDtype kv, hipStream_t stream) {
  if (!attention_supported(a.hq, a.hkv, a.d) || a.splits <= 0 || a.batch <= 0) return hipErrorInvalidValue;
  if (a.qkv_parts < 1 || a.qkv_parts > (a.page_table ? kAttnMaxQkvParts : 1)) return hipErrorInvalidValue;
  if (!a.page_table && a.batch != 1) return hipErrorInvalidValue;  // the contiguous cache holds one sequence
  // The interleave rule (page i of sequence b is i * page_interleave + b)
  // needs a table it describes and one page per sequence per index.
  if (a.page_interleave < 0 || (a.page_interleave > 0 && (!a.page_table || a.page_interleave < a.batch)))
    return hipErrorInvalidValue;
  if (a.batch > 1 && (a.part_stride < static_cast<int64_t>(attention_partial_floats(a.hq, a.hkv, a.d, a.splits)) ||
                      (mode == kAttnFused && a.qkv_stride <= 0)))
    return hipErrorInvalidValue;
  return kv == kKvF16 ? launch_attn_kv<__half>(a, mode, stream) : launch_attn_kv<float>(a, mode, stream);
}

hipError_t launch_attention_combine(const float* part, int hq, int hkv, int d, int splits, float* out,
                                    hipStream_t stream, int batch, int64_t part_stride, const L2WarmSet* warm) {
  if (!attention_supported(hq, hkv, d) || d > 128 || splits <= 0 || splits > kCombineKernelMaxSplits || batch <= 0)
    return hipErrorInvalidValue;
  const int nslice = (d + kCombineSlice - 1) / kCombineSlice;
  L2WarmSet w;
  int blocks = hq * nslice;
  if (warm && warm->blocks > 0) {
    if (batch != 1 || warm->blocks % kXcds != 0) return hipErrorInvalidValue;
    w = *warm;
    blocks = (blocks + kXcds - 1) / kXcds * kXcds + w.blocks;
  }
  const dim3 grid(blocks, batch);
  // Rounds of loads per thread: the smallest instantiated count that covers
  // the splits, so few of a thread's loads are clamped repeats (weight 0).
  const int rounds = (splits + kCombineGroups - 1) / kCombineGroups;
#define MMR_COMBINE_ROUNDS(K)                                                                                      \
  if (rounds <= K) {                                                                                               \
    attention_combine_kernel<K, false><<<grid, kCombineThreads, 0, stream>>>(part, hq, hkv, d, splits, part_stride, \
                                                                             out, w);                              \
    return hipGetLastError();                                                                                      \
  }
  MMR_COMBINE_ROUNDS(2)
  MMR_COMBINE_ROUNDS(4)
  MMR_COMBINE_ROUNDS(6)
  MMR_COMBINE_ROUNDS(8)
  MMR_COMBINE_ROUNDS(10)
  MMR_COMBINE_ROUNDS(12)
  MMR_COMBINE_ROUNDS(14)
  MMR_COMBINE_ROUNDS(16)
  MMR_COMBINE_ROUNDS(20)
  MMR_COMBINE_ROUNDS(24)
  MMR_COMBINE_ROUNDS(28)
  MMR_COMBINE_ROUNDS(32)
#undef MMR_COMBINE_ROUNDS
  attention_combine_kernel<16, true><<<grid, kCombineThreads, 0, stream>>>(part, hq, hkv, d, splits, part_stride, out,
                                                                           w);
  return hipGetLastError();
}

hipError_t launch_qkv_postprocess(const QkvPostArgs& a, KvDtype kv, hipStream_t stream) {
  if (!attention_supported(a.hq, a.hkv, a.d)) return hipErrorInvalidValue;
  return kv == kKvF16 ? launch_post_kv<__half>(a, stream) : launch_post_kv<float>(a, stream);
}

}  // namespace mmr
