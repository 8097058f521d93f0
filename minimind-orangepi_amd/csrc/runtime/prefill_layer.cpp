#include "prefill_layer.h"

#include "device.h"

#include <algorithm>
#include <stdexcept>

namespace minimind::model {

namespace {

// Slices of a scratch in carve order; `take` walks them over a base pointer
// (nullptr: sizing only).
struct Carver {
  char* base = nullptr;
  std::size_t used = 0;
  template <typename T>
  T* take(int64_t count) {
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += Arena::round_up(static_cast<std::size_t>(count) * sizeof(T));
    return p;
  }
};

PrefillScratch carve(const MiniMindConfig& c, int64_t rows, Carver& cv) {
  const int64_t H = c.hidden_size, D = c.head_dim, Hq = c.num_attention_heads, F = c.intermediate_size;
  auto planes = [&](int64_t cols, int chunk) {
    mmr::SplitPlanes p;
    p.hi = cv.take<uint16_t>(rows * cols);
    p.lo = cv.take<uint16_t>(rows * cols);
    p.inv = cv.take<float>(rows * ((cols + chunk - 1) / chunk));
    p.chunk = chunk;
    return p;
  };
  PrefillScratch s;
  s.rows = rows;
  s.x = cv.take<float>(rows * H);
  s.q = cv.take<float>(rows * Hq * D);
  s.attn = cv.take<float>(rows * Hq * D);
  s.part_floats = prefill_partial_floats(c, rows);
  s.part = cv.take<float>(s.part_floats);
  s.act = cv.take<float>(rows * F);
  s.xs = planes(H, mmr::kSplitChunk);
  s.attn_s = planes(Hq * D, mmr::kSplitChunkFine);
  s.act_s = planes(F, mmr::kSplitChunkFine);
  return s;
}

// Which inputs the GEMMs take pre-split for this row count.
struct SplitChoice {
  bool x = false, attn = false, act = false;
};
SplitChoice split_choice(const MiniMindConfig& c, int rows) {
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int Hq = static_cast<int>(c.num_attention_heads), Hkv = static_cast<int>(c.num_key_value_heads);
  const int F = static_cast<int>(c.intermediate_size);
  const int qkv_w = (Hq + 2 * Hkv) * D;
  SplitChoice sc;
  // The normalised rows go to the QKV and gate_up GEMMs pre-split when the
  // tiled path takes them (all but the few-rows path): the GEMM blocks then
  // stage the planes instead of each splitting the same rows again.
  sc.x = mmr::gemm_presplit_supported(rows, qkv_w, H) && mmr::gemm_presplit_supported(rows, 2 * F, H);
  // Likewise the attention output (written split by the attention kernel)
  // for the O GEMM, and act (written split by the gate_up SwiGLU epilogue)
  // for the down GEMM.
  sc.attn = D % mmr::kSplitChunkFine == 0 && mmr::gemm_presplit_supported(rows, H, Hq * D);
  sc.act = mmr::gemm_swiglu_split_supported(rows, 2 * F, H) && mmr::gemm_presplit_supported(rows, H, F);
  return sc;
}

}  // namespace

std::size_t prefill_scratch_bytes(const MiniMindConfig& c, int64_t rows) {
  Carver cv;
  (void)carve(c, rows, cv);
  return cv.used;
}

PrefillScratch carve_prefill_scratch(const MiniMindConfig& c, int64_t rows, void* base) {
  if (!base) throw std::invalid_argument("null prefill scratch");
  Carver cv;
  cv.base = static_cast<char*>(base);
  return carve(c, rows, cv);
}

void enqueue_prefill_input_norm(const MiniMindConfig& c, const PrefillScratch& s, int rows, const float* h,
                                const float* norm, hipStream_t stream) {
  const SplitChoice sc = split_choice(c, rows);
  check_hip(mmr::launch_batch_residual_norm(const_cast<float*>(h), nullptr, 0, rows, static_cast<int>(c.hidden_size),
                                            norm, c.rms_norm_eps, sc.x ? nullptr : s.x, false, stream,
                                            sc.x ? &s.xs : nullptr),
            "prefill input norm");
}

void enqueue_prefill_layer(const MiniMindConfig& c, const LayerDev& w, const float* inv_freq, const PrefillScratch& s,
                           const PrefillKv& kv, int rows, float* h, const float* next_norm, bool final_norm,
                           hipStream_t stream) {
  if (rows <= 0 || rows > s.rows) throw std::invalid_argument("prefill rows exceed the scratch");
  const int H = static_cast<int>(c.hidden_size), D = static_cast<int>(c.head_dim);
  const int Hq = static_cast<int>(c.num_attention_heads), Hkv = static_cast<int>(c.num_key_value_heads);
  const int F = static_cast<int>(c.intermediate_size);
  const int qkv_w = (Hq + 2 * Hkv) * D;
  const SplitChoice sc = split_choice(c, rows);
  float* const xf = sc.x ? nullptr : s.x;  // fp32 normalised rows, when the GEMMs read those
  const mmr::SplitPlanes* xs = sc.x ? &s.xs : nullptr;
  auto use_planes = [](mmr::GemmArgs& g, const mmr::SplitPlanes& p) {
    g.a = nullptr;
    g.a_hi = p.hi;
    g.a_lo = p.lo;
    g.a_inv = p.inv;
    g.a_chunk = p.chunk;
  };
  auto use_x = [&](mmr::GemmArgs& g) {
    if (sc.x) {
      use_planes(g, s.xs);
    } else {
      g.a = s.x;
    }
  };
  // Split-K partial products into s.part (at most max_splits; returns the
  // split count, 1 = the dense product); the consumers add the partials:
  // q/k norm + RoPE + KV write, residual add + RMSNorm, or SwiGLU.
  auto gemm_parts = [&](const float* a, int lda, const __half* wm, int N, int K, int max_splits) {
    mmr::GemmArgs g;
    if (a == s.x) {
      use_x(g);
    } else if (a == s.attn && sc.attn) {
      use_planes(g, s.attn_s);
    } else if (a == s.act && sc.act) {
      use_planes(g, s.act_s);
    } else {
      g.a = a;
    }
    g.lda = lda;
    g.w = wm;
    g.c = s.part;
    g.ldc = N;
    g.m = rows;
    g.n = N;
    g.k = K;
    g.k_splits = std::min(mmr::gemm_k_splits(rows, N, K), max_splits);
    g.split_stride = static_cast<int64_t>(rows) * N;
    g.register_staged = s.register_staged;
    if (int64_t{g.k_splits} * g.split_stride > s.part_floats)
      throw std::logic_error("prefill split-K partials exceed their buffer");
    check_hip(mmr::launch_gemm(g, stream), "prefill gemm");
    return g.k_splits;
  };
  constexpr int kAnySplits = 1 << 30;

  const int sq = gemm_parts(s.x, H, w.qkv, qkv_w, H, mmr::kQkvRowsMaxParts);
  mmr::QkvRowsArgs q;
  q.qkv = s.part;
  q.qkv_stride = qkv_w;
  q.qkv_parts = sq;
  q.qkv_part_stride = static_cast<int64_t>(rows) * qkv_w;
  q.q_norm = w.q_norm;
  q.k_norm = w.k_norm;
  q.eps = c.rms_norm_eps;
  q.inv_freq = inv_freq;
  q.start = kv.rope_start;
  q.row0 = kv.row0;
  q.tokens = rows;
  q.seg = kv.seg;
  q.hq = Hq;
  q.hkv = Hkv;
  q.d = D;
  q.query = s.q;
  q.query_stride = Hq * D;
  check_hip(mmr::launch_qkv_rows(q, kv.dtype, stream), "prefill qkv rows");
  mmr::PrefillAttnArgs at;
  at.query = s.q;
  at.query_stride = Hq * D;
  at.seg = kv.seg;
  at.start = kv.row0;
  at.tokens = rows;
  at.hq = Hq;
  at.hkv = Hkv;
  at.d = D;
  at.out = sc.attn ? nullptr : s.attn;
  at.out_stride = Hq * D;
  if (sc.attn) at.out_split = s.attn_s;
  check_hip(mmr::launch_prefill_attention(at, kv.dtype, stream), "prefill attention");
  const int so = gemm_parts(s.attn, Hq * D, w.o, H, Hq * D, kAnySplits);
  check_hip(mmr::launch_batch_residual_norm(h, s.part, so, rows, H, w.post_norm, c.rms_norm_eps, xf, false, stream, xs),
            "prefill residual + post norm");
  if (mmr::gemm_swiglu_supported(rows, 2 * F, H)) {  // SwiGLU in the gate_up epilogue
    mmr::GemmArgs g;
    use_x(g);
    g.lda = H;
    g.w = w.gate_up;
    g.c = sc.act ? nullptr : s.act;
    if (sc.act) g.act_split = s.act_s;
    g.ldc = F;
    g.m = rows;
    g.n = 2 * F;
    g.k = H;
    g.swiglu = true;
    g.register_staged = s.register_staged;
    check_hip(mmr::launch_gemm(g, stream), "prefill gate_up + SwiGLU");
  } else {
    const int sg = gemm_parts(s.x, H, w.gate_up, 2 * F, H, kAnySplits);
    check_hip(mmr::launch_batch_swiglu(s.part, sg, rows, F, s.act, stream), "prefill swiglu");
  }
  const int sd = gemm_parts(s.act, F, w.down, H, F, kAnySplits);
  // The next layer's input norm, or the final norm, whose rows are not split
  // (nothing multiplies them: the head normalises the last row itself).
  check_hip(mmr::launch_batch_residual_norm(h, s.part, sd, rows, H, next_norm, c.rms_norm_eps,
                                            final_norm ? s.x : xf, final_norm, stream, final_norm ? nullptr : xs),
            "prefill residual + norm");
}

}  // namespace minimind::model
