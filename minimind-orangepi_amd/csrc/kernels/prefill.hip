// prefill.hip -- prompt (prefill) kernels for gfx950: fp16-weight GEMM on the
// fp16 matrix cores (hi/lo split of the fp32 activations), per-row q/k norm +
// RoPE + KV-cache write, interleaved SwiGLU rows, and causal attention over
// the cache on the matrix cores (fp16 with hi/lo q and p for an fp16 cache,
// fp32 for an fp32 cache).
//
// Replaces the reference's device prefill layer (run_dense_prefill_layer_device,
// decoder_layer.cpp:661-734): device_matmul / device_matmul_add with batch =
// seq_len (ascend_matmul.h:102-107, aclnnMm at ascend_matmul.cpp:553-556),
// device_qkv_split_rows + q/k device_rms_norm_rows + device_rope_rows
// (ascend_custom_ops.h:80-107), device_prefill_attention (ascend_custom_ops.h:
// 122-130, kernel K8) and device_swiglu_rows.  The CPU semantics being matched
// are those of token-by-token decode (decoder_layer.cpp:312-407), which is what
// the reference runs on the CPU for a prompt (language_model.cpp:384-386).
//
// GEMM: C[m][n] (+)= sum_k A[m][k] * W[n][k], A fp32 row-major, W fp16
// row-major (the decode GEMVs' weights), fp32 accumulation.  W is exact in
// fp16; each K tile of A is split into hi + lo fp16 planes under a
// power-of-two row scale, which keeps ~22 significant bits (fp32 has 24), so
// the products on v_mfma_f32_16x16x32_f16 are as exact as the CPU path's.
// A 256-thread block computes a BM x BN tile with 2 x 2 waves; K advances 128
// at a time through LDS rows padded to 136 halves, which makes the 16-byte
// fragment reads of 16 lanes hit 64 distinct banks.
#include "device_common.h"
#include "kernels.h"

#include <algorithm>
#include <type_traits>

namespace mmr {
namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));

// One 16-byte KV chunk (8 fp16 or 4 fp32 values) -> fp32.
template <typename KV>
__device__ __forceinline__ void chunk_to_float_n(const uint4& c, float* f);
template <>
__device__ __forceinline__ void chunk_to_float_n<__half>(const uint4& c, float* f) {
  half8_to_float8(c, f);
}
template <>
__device__ __forceinline__ void chunk_to_float_n<float>(const uint4& c, float* f) {
  f[0] = __uint_as_float(c.x);
  f[1] = __uint_as_float(c.y);
  f[2] = __uint_as_float(c.z);
  f[3] = __uint_as_float(c.w);
}

constexpr int kGemmThreads = 256;
constexpr int kGemmBK = 128;           // K per LDS tile: the next tile's loads overlap this tile's MFMAs
constexpr int kGemmLDH = kGemmBK + 8;  // halves per LDS row (16-byte aligned, conflict-free fragment reads)

using f16x8 = _Float16 __attribute__((ext_vector_type(8)));
using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using f16x4 = _Float16 __attribute__((ext_vector_type(4)));
using i16x4 = short __attribute__((ext_vector_type(4)));

// Per-thread staging registers of one K tile: BM x BK fp32 of A as float4s,
// BN x BK fp16 of W as 8-half chunks; thread t takes chunks t, t + 256, ...
// so consecutive lanes read consecutive 16-byte pieces of a row (32 lanes per
// A row, 16 per W row).
// How a GEMM block gets A: fp32 rows it splits itself (kSplitNone); planes
// pre-split per 128 columns, one scale per row and K tile (kSplitTile); planes
// pre-split per 32 columns, brought to one scale per row and K tile while
// staging (kSplitFine).
constexpr int kSplitNone = 0, kSplitTile = 1, kSplitFine = 2;

template <int BM, int BN, int kMode = kSplitNone>
struct GemmStage {
  static constexpr bool kPreSplit = kMode != kSplitNone;
  static constexpr int kA = BM * kGemmBK / 4 / kGemmThreads;
  static constexpr int kB = BN * kGemmBK / 8 / kGemmThreads;
  // Pre-split A: 16-byte chunks (8 halves) of each plane per thread.
  static constexpr int kP = kPreSplit ? BM * kGemmBK / 8 / kGemmThreads : 1;
  float4 a[kPreSplit ? 1 : kA];
  uint4 ph[kP], pl[kP];
  // kSplitTile: row tid's scale; kSplitFine: the scale of each chunk's 32 columns.
  float pinv[kMode == kSplitFine ? kP : 1];
  uint4 b[kB];

  __device__ __forceinline__ void load(const GemmArgs& g, int m0, int n0, int k0, int tid) {
    if constexpr (kPreSplit) {
      static_assert(kP >= 1 && BM <= kGemmThreads, "tile too small for the block");
      static_assert(kGemmBK == kSplitChunk && kGemmBK % kSplitChunkFine == 0, "scale layout");
#pragma unroll
      for (int i = 0; i < kP; ++i) {
        const int idx = tid + i * kGemmThreads;
        const int r = idx / (kGemmBK / 8), q = idx % (kGemmBK / 8);
        const int row = min(m0 + r, g.m - 1);  // clamped: in bounds, never stored
        const int kc = k0 + q * 8;               // past k (last, partial tile): clamped load, zeroed
        const int64_t off = static_cast<int64_t>(row) * g.lda + min(kc, g.k - 8);
        const uint4 vh = *reinterpret_cast<const uint4*>(g.a_hi + off);
        const uint4 vl = *reinterpret_cast<const uint4*>(g.a_lo + off);
        ph[i] = kc < g.k ? vh : make_uint4(0u, 0u, 0u, 0u);
        pl[i] = kc < g.k ? vl : make_uint4(0u, 0u, 0u, 0u);
      }
      if constexpr (kMode == kSplitTile) {
        const int nkc = (g.k + kGemmBK - 1) / kGemmBK;
        pinv[0] = g.a_inv[static_cast<int64_t>(min(m0 + min(tid, BM - 1), g.m - 1)) * nkc + k0 / kGemmBK];
      } else {
        const int nkc = (g.k + kSplitChunkFine - 1) / kSplitChunkFine;
#pragma unroll
        for (int i = 0; i < kP; ++i) {
          const int idx = tid + i * kGemmThreads;
          const int r = idx / (kGemmBK / 8), q = idx % (kGemmBK / 8);
          const int c = min((k0 + q * 8) / kSplitChunkFine, nkc - 1);  // past k: any scale, the planes are zero
          pinv[i] = g.a_inv[static_cast<int64_t>(min(m0 + r, g.m - 1)) * nkc + c];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kA; ++i) {
        const int idx = tid + i * kGemmThreads;
        const int r = idx / (kGemmBK / 4), q = idx % (kGemmBK / 4);
        const int row = min(m0 + r, g.m - 1);  // clamped: in bounds, never stored
        const int kc = k0 + q * 4;               // past k (last, partial tile): clamped load, zeroed
        const float4 v = *reinterpret_cast<const float4*>(g.a + static_cast<int64_t>(row) * g.lda + min(kc, g.k - 4));
        a[i] = kc < g.k ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int idx = tid + i * kGemmThreads;
      const int r = idx / (kGemmBK / 8), q = idx % (kGemmBK / 8);
      const int row = min(n0 + r, g.n - 1);
      const int kc = k0 + q * 8;
      const uint4 v = *reinterpret_cast<const uint4*>(g.w + static_cast<int64_t>(row) * g.k + min(kc, g.k - 8));
      b[i] = kc < g.k ? v : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  // A -> two fp16 planes with a power-of-two scale per row of the tile:
  // s = 2^(15 - e) for the row's max |a| = f 2^e (f in [1/2, 1)), hi =
  // fp16(s a), lo = fp16(s a - hi) (the subtraction is exact), inv[r] = 1/s.
  // The 32 lanes holding a row reduce its maximum together.
  __device__ __forceinline__ void store(_Float16 (*Ah)[kGemmLDH], _Float16 (*Al)[kGemmLDH], float* inv,
                                        _Float16 (*Bs)[kGemmLDH], int tid) const {
    if constexpr (kMode == kSplitTile) {
#pragma unroll
      for (int i = 0; i < kP; ++i) {
        const int idx = tid + i * kGemmThreads;
        const int r = idx / (kGemmBK / 8), q = idx % (kGemmBK / 8);
        *reinterpret_cast<uint4*>(&Ah[r][q * 8]) = ph[i];
        *reinterpret_cast<uint4*>(&Al[r][q * 8]) = pl[i];
      }
      if (tid < BM) inv[tid] = pinv[0];
    } else if constexpr (kMode == kSplitFine) {
      // The 16 lanes holding a row's tile take its largest chunk scale as the
      // tile's, and multiply their chunk by the power of two between the two
      // (exact but for results below fp16's normal range, i.e. below 2^-29 of
      // the tile's largest value: far under fp32 accumulation's rounding).
#pragma unroll
      for (int i = 0; i < kP; ++i) {
        const int idx = tid + i * kGemmThreads;
        const int r = idx / (kGemmBK / 8), q = idx % (kGemmBK / 8);
        const float tinv = group_max<kGemmBK / 8>(pinv[i]);
        int ec = 0, et = 0;
        frexpf(pinv[i], &ec);
        frexpf(tinv, &et);
        const _Float16 ratio = static_cast<_Float16>(ldexpf(1.0f, ec - et));  // 2^-d, 0 below 2^-24
        f16x8 vh, vl;
        __builtin_memcpy(&vh, &ph[i], 16);
        __builtin_memcpy(&vl, &pl[i], 16);
        vh *= ratio;
        vl *= ratio;
        *reinterpret_cast<f16x8*>(&Ah[r][q * 8]) = vh;
        *reinterpret_cast<f16x8*>(&Al[r][q * 8]) = vl;
        if (q == 0) inv[r] = tinv;
      }
    }
#pragma unroll
    for (int i = 0; i < (kPreSplit ? 0 : kA); ++i) {
      const int idx = tid + i * kGemmThreads;
      const int r = idx / (kGemmBK / 4), q = idx % (kGemmBK / 4);
      const float4 v = a[i];
      const float mx = group_max<32>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
      int e = 0;
      frexpf(mx, &e);  // e = 0 for a zero row
      e = max(e, -100);
      const float sc = ldexpf(1.0f, 15 - e);
      const float x[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
      f16x4 hi, lo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[j] = static_cast<_Float16>(x[j]);
        lo[j] = static_cast<_Float16>(x[j] - static_cast<float>(hi[j]));
      }
      *reinterpret_cast<f16x4*>(&Ah[r][q * 4]) = hi;
      *reinterpret_cast<f16x4*>(&Al[r][q * 4]) = lo;
      if (q == 0) inv[r] = ldexpf(1.0f, e - 15);
    }
#pragma unroll
    for (int i = 0; i < kB; ++i) {
      const int idx = tid + i * kGemmThreads;
      const int r = idx / (kGemmBK / 8), q = idx % (kGemmBK / 8);
      *reinterpret_cast<uint4*>(&Bs[r][q * 8]) = b[i];
    }
  }
};

// C[m][n] (+)= sum_k A[m][k] W[n][k] for a BM x BN tile per block of 4 waves
// (2 x 2, each BM/2 x BN/2 of 16 x 16 fragments), on the fp16 matrix cores.
// Per K tile: MFMA v_mfma_f32_16x16x32_f16 over the hi and lo planes of A
// (lane l supplies A row l % 16 and W row l % 16 at the same 8 k positions
// 8 (l / 16) ..), the products are exact and summed in fp32, then the tile's
// sum is scaled by the row's 1/s (exact) into the accumulator.  W is exact in
// fp16; hi + lo carries ~22 significant bits of each activation.  The LDS
// footprint (~52 KB for 64 x 64) lets two or three blocks share a CU, which
// hides one block's tile-load wait behind another's work.
// Epilogues of gemm_f16w_kernel: store C; add the residual; SwiGLU over the
// interleaved gate/up columns (2i, 2i + 1) -> act[m][i] (decoder_layer.cpp:
// 175-182), the pair meeting through one lane exchange.
constexpr int kGemmEpiStore = 0, kGemmEpiResidual = 1, kGemmEpiSwiGlu = 2;

// Epilogue shared by the GEMM kernels: the block's accumulators (BM x BN, 2 x
// 2 waves of 16 x 16 fragments; lane holds rows 4 (lane / 16) + {0..3} of
// column lane % 16 of each fragment) go to C (store / + residual), or through
// SwiGLU to act, optionally pre-split.  act_scratch: LDS the K loop no longer
// uses, at least BM x (BN / 2 + 4) floats.
template <int BM, int BN, int kEpi>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, const f32x4 (&acc)[BM / 32][BN / 32], float* out,
                                              float* act_scratch, int m0, int n0, int tid) {
  constexpr bool kResidual = kEpi == kGemmEpiResidual;
  constexpr int TM = BM / 32, TN = BN / 32;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wm = wave / 2, wn = wave % 2;
  // Output fragment: lane holds rows 4 * (lane / 16) + {0..3} of column
  // lane % 16 of each 16 x 16 tile.  Residual loads are issued together
  // (clamped indices), then the in-range elements are stored.
  float res[TM][TN][4];
  if constexpr (kResidual) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = min(n0 + wn * (BN / 2) + j * 16 + lane % 16, g.n - 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = min(m0 + wm * (BM / 2) + i * 16 + 4 * (lane / 16) + r, g.m - 1);
          res[i][j][r] = g.residual[static_cast<int64_t>(row) * g.ldc + col];
        }
      }
  }
  // SwiGLU over lane pairs: lane 2c holds gate column 2c and lane 2c + 1 up
  // column 2c + 1, of the same four rows 4 (lane / 16) + r.  One neighbour
  // exchange per row, then the even lane forms act for rows r = 0, 1 and the
  // odd lane for r = 2, 3: two SwiGLUs per lane and fragment, not four.
  // Output k of this lane is row rsw[k] of the fragment.
  const bool odd = (lane & 1) != 0;
  const int rsw[2] = {odd ? 2 : 0, odd ? 3 : 1};
  auto swiglu_pair = [&](const f32x4& v, float (&act)[2]) {
    const float x0 = dpp_move<dpp::kQuadXor1>(v[0]), x1 = dpp_move<dpp::kQuadXor1>(v[1]);
    const float x2 = dpp_move<dpp::kQuadXor1>(v[2]), x3 = dpp_move<dpp::kQuadXor1>(v[3]);
    const float gate[2] = {odd ? x2 : v[0], odd ? x3 : v[1]};
    const float up[2] = {odd ? v[2] : x0, odd ? v[3] : x1};
#pragma unroll
    for (int k = 0; k < 2; ++k) act[k] = silu_fast(gate[k]) * up[k];
  };
  bool act_to_lds = false;
  constexpr bool kActSplit = kEpi == kGemmEpiSwiGlu && (BN == 128 || BN == 64);  // whole 32-column act chunks
  constexpr int kActLd = BN / 2 + 4;  // floats per row of the act tile in LDS
  if constexpr (kActSplit) act_to_lds = g.act_split.hi != nullptr;
  if (act_to_lds) {
    // act tile for the pre-split writer below: [BM][BN / 2] (padded) over the
    // W staging buffer, which the K loop no longer reads.  Rows past m hold
    // values of clamped rows; the writer skips them.
    float* act_s = act_scratch;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float act[2];
        swiglu_pair(acc[i][j], act);
#pragma unroll
        for (int k = 0; k < 2; ++k)
          act_s[(wm * (BM / 2) + i * 16 + 4 * (lane / 16) + rsw[k]) * kActLd + (wn * (BN / 2) + j * 16 + lane % 16) / 2] =
              act[k];
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * (BN / 2) + j * 16 + lane % 16;
        if constexpr (kEpi == kGemmEpiSwiGlu) {
          float act[2];
          swiglu_pair(acc[i][j], act);
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int row = m0 + wm * (BM / 2) + i * 16 + 4 * (lane / 16) + rsw[k];
            if (row < g.m && col < g.n) out[static_cast<int64_t>(row) * g.ldc + col / 2] = act[k];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm * (BM / 2) + i * 16 + 4 * (lane / 16) + r;
            if (row < g.m && col < g.n)
              out[static_cast<int64_t>(row) * g.ldc + col] = kResidual ? res[i][j][r] + acc[i][j][r] : acc[i][j][r];
          }
        }
      }
  }
  if constexpr (kActSplit) {
    if (act_to_lds) {
      // act pre-split per 32 columns (the down GEMM's A): thread = 4
      // consecutive columns of one row, the 8 threads of a chunk reduce its
      // max together, then write 8-byte runs of both planes.
      __syncthreads();
      const float* act_s = act_scratch;
      const int nkc = g.n / 2 / kSplitChunkFine;
#pragma unroll
      for (int p = 0; p < BM * (BN / 2) / 4 / kGemmThreads; ++p) {
        const int idx = tid + p * kGemmThreads;
        const int r = idx / (BN / 8), c4 = idx % (BN / 8);
        const int row = m0 + r, col = n0 / 2 + c4 * 4;
        const bool ok = row < g.m && col < g.n / 2;
        const float4 v = ok ? *reinterpret_cast<const float4*>(&act_s[r * kActLd + c4 * 4])
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float mx =
            group_max<kSplitChunkFine / 4>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        int e = 0;
        frexpf(mx, &e);  // e = 0 for a zero chunk
        e = max(e, -100);
        const float sc = ldexpf(1.0f, 15 - e);
        const float x[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
        f16x4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          hi[j] = static_cast<_Float16>(x[j]);
          lo[j] = static_cast<_Float16>(x[j] - static_cast<float>(hi[j]));
        }
        if (ok) {
          const int64_t off = static_cast<int64_t>(row) * g.ldc + col;
          *reinterpret_cast<f16x4*>(g.act_split.hi + off) = hi;
          *reinterpret_cast<f16x4*>(g.act_split.lo + off) = lo;
          if (c4 % (kSplitChunkFine / 4) == 0)
            g.act_split.inv[static_cast<int64_t>(row) * nkc + col / kSplitChunkFine] = ldexpf(1.0f, e - 15);
        }
      }
    }
  }
}

template <int BM, int BN, int kEpi, int kMode>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_f16w_kernel(GemmArgs g) {
  constexpr int TM = BM / 32, TN = BN / 32;  // 16 x 16 MFMA tiles per wave
  static_assert(GemmStage<BM, BN>::kA >= 1 && GemmStage<BM, BN>::kB >= 1, "tile too small for the block");
  __shared__ __align__(16) _Float16 Ah[BM][kGemmLDH];
  __shared__ __align__(16) _Float16 Al[BM][kGemmLDH];
  __shared__ __align__(16) _Float16 Bs[BN][kGemmLDH];
  __shared__ __align__(16) float inv_s[BM];
  static_assert(BM * (BN / 2 + 4) * 4 <= BN * kGemmLDH * 2, "act tile exceeds the W buffer");
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Split z (grid z) takes K tiles [kt0, kt1); an empty range writes zeros.
  const int nk = (g.k + kGemmBK - 1) / kGemmBK;
  const int per = (nk + static_cast<int>(gridDim.z) - 1) / static_cast<int>(gridDim.z);
  const int kt0 = static_cast<int>(blockIdx.z) * per, kt1 = min(kt0 + per, nk);
  float* out = g.c + static_cast<int64_t>(blockIdx.z) * g.split_stride;

  GemmStage<BM, BN, kMode> stage;
  stage.load(g, m0, n0, kt0 * kGemmBK, tid);  // past k: clamped loads, zeroed
  stage.store(Ah, Al, inv_s, Bs, tid);
  __syncthreads();
  for (int kt = kt0; kt < kt1; ++kt) {
    // The next tile's loads are in flight during this tile's MFMAs; on the
    // last tile they reload it (unconditional, so the values stay in registers).
    stage.load(g, m0, n0, min(kt + 1, kt1 - 1) * kGemmBK, tid);
    f32x4 part[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) part[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < kGemmBK; kb += 32) {
      const int kk = kb + 8 * (lane / 16);
      f16x8 ah[TM], al[TM], bw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        ah[i] = *reinterpret_cast<const f16x8*>(&Ah[wm * (BM / 2) + i * 16 + lane % 16][kk]);
        al[i] = *reinterpret_cast<const f16x8*>(&Al[wm * (BM / 2) + i * 16 + lane % 16][kk]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) bw[j] = *reinterpret_cast<const f16x8*>(&Bs[wn * (BN / 2) + j * 16 + lane % 16][kk]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bw[j], part[i][j], 0, 0, 0);
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bw[j], part[i][j], 0, 0, 0);
        }
    }
    // Output rows of lane: 4 (lane / 16) + r of each 16-row fragment.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const float4 sv = *reinterpret_cast<const float4*>(&inv_s[wm * (BM / 2) + i * 16 + 4 * (lane / 16)]);
      const float sr[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(part[i][j][r], sr[r], acc[i][j][r]);
    }
    __syncthreads();
    stage.store(Ah, Al, inv_s, Bs, tid);
    __syncthreads();
  }

  gemm_epilogue<BM, BN, kEpi>(g, acc, out, reinterpret_cast<float*>(&Bs[0][0]), m0, n0, tid);
}

// ---- GEMM with direct global->LDS loads (pre-split A, K % 64 == 0) ----
// The same product as gemm_f16w_kernel with A given as fp16 hi/lo planes,
// but the tiles never pass through registers: every 16-byte piece of a K
// tile goes from global memory straight into LDS (global_load_lds_dwordx4),
// and three 64-wide K stages are in flight, so a block keeps up to two tiles
// loading while it multiplies the third (the register-staged kernel has one).
// The loads write 64 lanes x 16 bytes contiguously; the LDS image of a stage
// is [rows][8 chunks of 8 halves] with chunk kc of row r at position
// r * 8 + (kc ^ ((r >> 1) & 7)), so the matrix cores' fragment reads (16
// lanes = 16 rows at one chunk) touch 16 distinct 16-byte bank groups.  The
// row scales (one per row and 128 columns, or per 32 columns) come through
// LDS the same way and are applied per stage, or per 32-k step.
constexpr int kDmaBK = 64;      // K per stage
constexpr int kDmaStages = 2;
constexpr int kDmaRowChunks = kDmaBK / 8;

__device__ __forceinline__ int dma_pos(int r, int kc) { return r * kDmaRowChunks + (kc ^ ((r >> 1) & 7)); }

// Wait until at most kPending of this thread's vector-memory operations are
// outstanding, then meet the other waves at a barrier.
template <int kPending>
__device__ __forceinline__ void dma_wait_barrier() {
  static_assert(kPending >= 0 && kPending < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(kPending) : "memory");
}

template <int BM, int BN, int kEpi, int kGran, int kStages = kDmaStages>
__global__ __launch_bounds__(kGemmThreads) void gemm_dma_kernel(GemmArgs g) {
  static_assert(kGran == kSplitChunk || kGran == kSplitChunkFine, "scale granularity");
  static_assert(kStages == 2, "the K loop is unrolled over the two stage buffers");
  constexpr int TM = BM / 32, TN = BN / 32;
  constexpr int kScales = kGran >= kDmaBK ? 1 : kDmaBK / kGran;  // scale values per row per stage
  constexpr int kAWaveLoads = BM * kDmaRowChunks / kWave / 4;  // per plane, per wave, per stage
  constexpr int kBWaveLoads = BN * kDmaRowChunks / kWave / 4;
  static_assert(kAWaveLoads >= 1 && kBWaveLoads >= 1 && BM <= kWave, "tile shape");
  __shared__ __align__(16) _Float16 Ah[kStages][BM * kDmaBK];
  __shared__ __align__(16) _Float16 Al[kStages][BM * kDmaBK];
  __shared__ __align__(16) _Float16 Bs[kStages][BN * kDmaBK];
  // Scales per stage, each wave its own copy (uniform op counts): [wave][s][row]
  __shared__ __align__(16) float Sc[kStages][4][kScales][kWave];
  static_assert(BM * (BN / 2 + 4) * 4 <= kStages * BN * kDmaBK * 2, "act tile exceeds the W stages");

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  // Wave-uniform (an SGPR): the LDS destinations of the direct loads are scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / 2, wn = wave % 2;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int nk = g.k / kDmaBK;
  const int per = (nk + static_cast<int>(gridDim.z) - 1) / static_cast<int>(gridDim.z);
  const int kt0 = static_cast<int>(blockIdx.z) * per, kt1 = min(kt0 + per, nk);
  float* out = g.c + static_cast<int64_t>(blockIdx.z) * g.split_stride;
  const int nsc = (g.k + kGran - 1) / kGran;  // scales per row of a_inv

  // This lane's byte offsets for the direct loads and its LDS fragment
  // offsets, the same for every stage: a stage only moves the scalar bases
  // and alternates the buffer (a constant offset, the loop being unrolled
  // over the two buffers).  Rows past m (n) load a clamped row: in bounds,
  // never stored.  (launch_gemm keeps every offset below 2^32.)
  uint32_t a_off[kAWaveLoads], b_off[kBWaveLoads];
#pragma unroll
  for (int j = 0; j < kAWaveLoads; ++j) {
    const int c = (wave + 4 * j) * kWave + lane;  // wave-wide load wave + 4 j fills chunks [64 i, 64 i + 64)
    const int r = c / kDmaRowChunks, kc = (c % kDmaRowChunks) ^ ((r >> 1) & 7);
    a_off[j] = static_cast<uint32_t>((static_cast<int64_t>(min(m0 + r, g.m - 1)) * g.lda + kc * 8) * 2);
  }
#pragma unroll
  for (int j = 0; j < kBWaveLoads; ++j) {
    const int c = (wave + 4 * j) * kWave + lane;
    const int r = c / kDmaRowChunks, kc = (c % kDmaRowChunks) ^ ((r >> 1) & 7);
    b_off[j] = static_cast<uint32_t>((static_cast<int64_t>(min(n0 + r, g.n - 1)) * g.k + kc * 8) * 2);
  }
  const uint32_t s_off = static_cast<uint32_t>(static_cast<int64_t>(min(m0 + min(lane, BM - 1), g.m - 1)) * nsc * 4);
  int a_rd[2][TM], b_rd[2][TN];  // [ks][fragment]: element offsets within a stage buffer
#pragma unroll
  for (int ks = 0; ks < kDmaBK / 32; ++ks) {
    const int kc = ks * 4 + lane / 16;
#pragma unroll
    for (int i = 0; i < TM; ++i) a_rd[ks][i] = dma_pos(wm * (BM / 2) + i * 16 + lane % 16, kc) * 8;
#pragma unroll
    for (int j = 0; j < TN; ++j) b_rd[ks][j] = dma_pos(wn * (BN / 2) + j * 16 + lane % 16, kc) * 8;
  }

  // Stage kt into buffer buf.
  auto issue = [&](int kt, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int64_t kb = static_cast<int64_t>(kt) * kDmaBK * 2;  // byte offset of the stage's first k
    const char* ahb = reinterpret_cast<const char*>(g.a_hi) + kb;
    const char* alb = reinterpret_cast<const char*>(g.a_lo) + kb;
    const char* wb = reinterpret_cast<const char*>(g.w) + kb;
#pragma unroll
    for (int j = 0; j < kAWaveLoads; ++j) {
      const int i = wave + 4 * j;
      dma_load<16>(ahb, a_off[j], lds_address(&Ah[buf][i * kWave * 8]));
      dma_load<16>(alb, a_off[j], lds_address(&Al[buf][i * kWave * 8]));
    }
#pragma unroll
    for (int j = 0; j < kBWaveLoads; ++j) {
      const int i = wave + 4 * j;
      dma_load<16>(wb, b_off[j], lds_address(&Bs[buf][i * kWave * 8]));
    }
#pragma unroll
    for (int sidx = 0; sidx < kScales; ++sidx)
      dma_load<4>(reinterpret_cast<const char*>(g.a_inv) + ((kt * kDmaBK + sidx * kGran) / kGran) * 4, s_off,
                  lds_address(&Sc[buf][wave][sidx][0]));
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // One K stage from buffer buf: wait for it, start the next one's loads
  // (none after the last stage: the direct loads are inline assembly, so the
  // block-uniform branch adds no compiler wait, and the epilogue waits for no
  // unused loads), then multiply.
  auto stage = [&](int kt, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    // Stage kt has landed, and every wave is done with the other buffer
    // (read in stage kt - 1).
    dma_wait_barrier<0>();
    if (kt + 1 < kt1) issue(kt + 1, std::integral_constant<int, buf ^ 1>{});
    f32x4 part[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) part[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < kDmaBK / 32; ++ks) {
      f16x8 ah[TM], al[TM], bw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        ah[i] = *reinterpret_cast<const f16x8*>(&Ah[buf][a_rd[ks][i]]);
        al[i] = *reinterpret_cast<const f16x8*>(&Al[buf][a_rd[ks][i]]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) bw[j] = *reinterpret_cast<const f16x8*>(&Bs[buf][b_rd[ks][j]]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bw[j], part[i][j], 0, 0, 0);
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bw[j], part[i][j], 0, 0, 0);
        }
      // Scale the finished k range by the rows' 1/s: every 32 k (fine
      // scales) or once per stage.
      if (kScales > 1 || ks == kDmaBK / 32 - 1) {
        const int sidx = kScales > 1 ? ks : 0;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const float4 sv = *reinterpret_cast<const float4*>(&Sc[buf][wave][sidx][wm * (BM / 2) + i * 16 + 4 * (lane / 16)]);
          const float sr[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
          for (int j = 0; j < TN; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(part[i][j][r], sr[r], acc[i][j][r]);
            part[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
        }
      }
    }
  };

  if (kt0 < kt1) {  // a split past the end of K writes zeros
    issue(kt0, std::integral_constant<int, 0>{});
    for (int kt = kt0; kt < kt1; kt += 2) {
      stage(kt, std::integral_constant<int, 0>{});
      if (kt + 1 < kt1) stage(kt + 1, std::integral_constant<int, 1>{});
    }
  }
  // Every wave is done with the stages before the epilogue reuses them.
  dma_wait_barrier<0>();
  gemm_epilogue<BM, BN, kEpi>(g, acc, out, reinterpret_cast<float*>(&Bs[0][0]), m0, n0, tid);
}

// Skinny GEMM for few rows of A (batched decode, m <= 16 * BT): one block per
// 16 rows of W, its kSkinnyWaves waves splitting K into contiguous ranges of
// 32-wide blocks.  Per 32-k block a lane loads 8 consecutive halves of W row
// n0 + lane % 16 and 8 fp32 of A row bt * 16 + lane % 16 at k offset
// 8 * (lane / 16); MFMA s (0..7) takes element s of both, so instruction s
// covers k = 8 g + s over the four lane groups g.  A wave issues the loads of
// up to kSkinnyGroup k-blocks before its first MFMA.  The waves' accumulators
// are summed in LDS in wave order (deterministic), then the residual epilogue.
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyGroup = 4;

template <int BT, bool kResidual>
__global__ __launch_bounds__(kWave* kSkinnyWaves) void gemm_skinny_kernel(GemmArgs g) {
  __shared__ __align__(16) float red[kSkinnyWaves][BT][kWave][4];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int n0 = blockIdx.x * 16;
  const int nblk = g.k / 32;
  const int b0 = wave * nblk / kSkinnyWaves, b1 = (wave + 1) * nblk / kSkinnyWaves;
  const int wrow = min(n0 + lane % 16, g.n - 1);
  const int koff = 8 * (lane / 16);
  const __half* wsrc = g.w + static_cast<int64_t>(wrow) * g.k + koff;
  const float* asrc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt)
    asrc[bt] = g.a + static_cast<int64_t>(min(bt * 16 + lane % 16, g.m - 1)) * g.lda + koff;

  f32x4 acc[BT];
#pragma unroll
  for (int bt = 0; bt < BT; ++bt) acc[bt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int kb = b0; kb < b1; kb += kSkinnyGroup) {
    uint4 wv[kSkinnyGroup];
    float4 av[kSkinnyGroup][BT][2];
#pragma unroll
    for (int i = 0; i < kSkinnyGroup; ++i) {
      const int blk = min(kb + i, b1 - 1);  // past the range: reload the last block, masked below
      wv[i] = *reinterpret_cast<const uint4*>(wsrc + blk * 32);
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        av[i][bt][0] = *reinterpret_cast<const float4*>(asrc[bt] + blk * 32);
        av[i][bt][1] = *reinterpret_cast<const float4*>(asrc[bt] + blk * 32 + 4);
      }
    }
#pragma unroll
    for (int i = 0; i < kSkinnyGroup; ++i) {
      if (kb + i < b1) {  // wave-uniform
        float wf[8];
        half8_to_float8(wv[i], wf);
#pragma unroll
        for (int bt = 0; bt < BT; ++bt) {
          const float a8[8] = {av[i][bt][0].x, av[i][bt][0].y, av[i][bt][0].z, av[i][bt][0].w,
                               av[i][bt][1].x, av[i][bt][1].y, av[i][bt][1].z, av[i][bt][1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[bt] = __builtin_amdgcn_mfma_f32_16x16x4f32(wf[e], a8[e], acc[bt], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int bt = 0; bt < BT; ++bt)
    *reinterpret_cast<f32x4*>(&red[wave][bt][lane][0]) = acc[bt];
  __syncthreads();
  // Output fragment of wave-lane l: rows n0 + 4 (l / 16) + r of W, column
  // (A row) bt * 16 + l % 16.  Threads split the BT * 64 * 4 outputs.
  for (int o = threadIdx.x; o < BT * kWave * 4; o += kWave * kSkinnyWaves) {
    const int bt = o / (kWave * 4), l = (o / 4) % kWave, r = o % 4;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) v += red[w][bt][l][r];
    const int n = n0 + 4 * (l / 16) + r;
    const int m = bt * 16 + l % 16;
    if (n < g.n && m < g.m) {
      const int64_t off = static_cast<int64_t>(m) * g.ldc + n;
      g.c[off] = kResidual ? g.residual[off] + v : v;
    }
  }
}

// Per (token, head) q/k RMSNorm + RoPE of one row of the fused qkv output,
// q to `query`, k/v rounded to the cache dtype and written at cache index
// start + token (decoder_layer.cpp:342-359 per token).  One wave per (head,
// token); a block holds kQkvRowsTokens consecutive tokens of one head, grid
// (hq + hkv, ceil(tokens / kQkvRowsTokens)).
constexpr int kQkvRowsTokens = 4;
template <typename KV, int D>
__global__ __launch_bounds__(kWave* kQkvRowsTokens) void qkv_rows_kernel(QkvRowsArgs a) {
  __shared__ float x_all[kQkvRowsTokens][D];
  const int b = blockIdx.x;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  // Wave = one token of the block's kQkvRowsTokens; past the last token the
  // wave works on a clamped row (every wave reaches the barriers) and stores
  // nothing.
  const int t_raw = blockIdx.y * kQkvRowsTokens + wave;
  const bool live = t_raw < a.tokens;
  const int t = min(t_raw, a.tokens - 1);
  float* x_s = x_all[wave];
  const bool is_q = b < a.hq;
  const int head = is_q ? b : b - a.hq;
  const float* row = a.qkv + static_cast<int64_t>(t) * a.qkv_stride;
  const float* src = row + (is_q ? head * D : a.hq * D + head * D);
  const float* vsrc = row + a.hq * D + a.hkv * D + head * D;
  const float* w = is_q ? a.q_norm : a.k_norm;
  const int d0 = min(lane, D - 1), d1 = min(lane + kWave, D - 1);
  // The projection's split partials at p[i]: every load of the wave (the q or
  // k row's partials, the V row's, the gains and the frequency) goes out
  // before any add; the partials are then added in split order, the clamped
  // duplicates past the last split as zeros (a select: a guarded add would be
  // a branch, with a wait and a reload inside it).
  using Parts = float[kQkvRowsMaxParts];
  auto part_load = [&](const float* p, int i, Parts& v) {
#pragma unroll
    for (int sp = 0; sp < kQkvRowsMaxParts; ++sp) v[sp] = p[min(sp, a.qkv_parts - 1) * a.qkv_part_stride + i];
  };
  auto part_add = [&](const Parts& v) {
    float x = v[0];
#pragma unroll
    for (int sp = 1; sp < kQkvRowsMaxParts; ++sp) x += sp < a.qkv_parts ? v[sp] : 0.0f;
    return x;
  };
  Parts px0, px1, pv0, pv1;
  part_load(src, d0, px0);
  part_load(src, d1, px1);
  // V rows of a KV head are loaded with the K rows (a query block's copy is unused).
  part_load(is_q ? src : vsrc, d0, pv0);
  part_load(is_q ? src : vsrc, d1, pv1);
  const float w0 = w[d0], w1 = w[d1];
  const float f = a.inv_freq[min(lane, D / 2 - 1)];
  asm volatile("" ::: "memory");
  float x0 = part_add(px0), x1 = part_add(px1);
  const float v0 = part_add(pv0), v1 = part_add(pv1);
  x0 = lane < D ? x0 : 0.0f;
  x1 = lane + kWave < D ? x1 : 0.0f;
  const float ss = group_sum<kWave>(x0 * x0 + x1 * x1);
  const float scale = __builtin_amdgcn_rsqf(fmaf(ss, 1.0f / static_cast<float>(D), a.eps));  // v_rsq_f32, about 1 ulp
  if (lane < D) x_s[lane] = x0 * (scale * w0);
  if (lane + kWave < D) x_s[lane + kWave] = x1 * (scale * w1);
  const int pos = a.start + t;
  float rc = 1.0f, rs = 0.0f;
  if (lane < D / 2) sincosf(static_cast<float>(pos) * f, &rs, &rc);
  __syncthreads();
  if (lane < D / 2) {
    const float first = x_s[lane];
    const float second = x_s[lane + D / 2];
    x_s[lane] = first * rc - second * rs;
    x_s[lane + D / 2] = second * rc + first * rs;
  }
  __syncthreads();
  if (!live) return;
  if (is_q) {
    float* dst = a.query + static_cast<int64_t>(t) * a.query_stride + head * D;
    for (int i = lane; i < D; i += kWave) dst[i] = x_s[i];
  } else {
    const int row = a.row0 + t;
    const int seg = kv_segment(row);
    const int64_t off = kv_segment_offset(seg, row, head, a.hkv, D);
    KV* kdst = static_cast<KV*>(a.seg.s[seg].k) + off;
    KV* vdst = static_cast<KV*>(a.seg.s[seg].v) + off;
    if (lane < D) {
      kdst[lane] = from_float<KV>(x_s[lane]);
      vdst[lane] = from_float<KV>(v0);
    }
    if (lane + kWave < D) {
      kdst[lane + kWave] = from_float<KV>(x_s[lane + kWave]);
      vdst[lane + kWave] = from_float<KV>(v1);
    }
  }
}

// Causal attention of `tokens` queries at positions start .. start + tokens - 1
// over the cache (keys 0 .. position of each query, decoder_layer.cpp:184-234
// per token), on the fp32 matrix cores (fp32 cache) or the fp16 ones (fp16
// cache, below).
//
// Block = (16 queries, one query head): 8 waves, wave w takes the 16-key tiles
// w, w + 8, ... of the block's causal range (two waves per SIMD, so one wave's
// vector work overlaps the other's matrix-core work), each with its own LDS stage (K and
// V row-major, loaded row-contiguously: consecutive lanes read consecutive 16
// bytes of one row) and its own online-softmax state, and fetches its next
// tile into registers while it computes the current one.  Per 16-key sub-tile
// a wave forms S^T = K Q^T (v_mfma_f32_16x16x4f32, D/16 slices x 4): lane l
// holds S^T[key 4(l/16)+i][query l%16], exactly the B-operand layout of
// O^T += V^T P^T (A = V^T: lane l reads V[key 4(l/16)+i][16j + l%16], four
// conflict-free LDS words), so the probabilities never move between lanes;
// only the per-query tile maximum needs the four 16-lane rows (two xor
// shuffles).
// Scores are dot / sqrt(d) in base-2 units (q pre-scaled by log2(e) / sqrt(d),
// softmax by exp2), masked above the query's position.  A wave may see tiles where a query has no key yet: its
// state stays (-inf, 0, 0) until one arrives.  At the end the waves' (m, l, O)
// merge in LDS (log-sum-exp, wave order): the per-query wave weights and 1/L
// are computed once, then each output is a dot product over the waves.
constexpr int kPrefillQueries = 16;
constexpr int kPrefillKeys = 16;  // keys per wave tile (one matrix-core sub-tile)
constexpr int kPrefillWaves = 8;

template <typename KV, int D>
struct PrefillTileRegs {
  static constexpr int CH = 16 / static_cast<int>(sizeof(KV));
  static constexpr int kChunks = kPrefillKeys * D / CH;  // 16-byte chunks of K (or V) per tile
  static constexpr int kPer = (kChunks + kWave - 1) / kWave;
  uint4 k[kPer], v[kPer];
};

template <typename KV, int D>
__global__ __launch_bounds__(kWave* kPrefillWaves) void prefill_attention_kernel(PrefillAttnArgs a) {
  using Regs = PrefillTileRegs<KV, D>;
  constexpr int CH = Regs::CH;
  constexpr int kChunks = Regs::kChunks;
  constexpr int kPer = Regs::kPer;
  constexpr int KT = kPrefillKeys;
  constexpr int LD = D + 4;    // K and V rows: 16-byte K fragment reads and the 4-row V reads hit distinct banks
  constexpr int DT = D / 16;   // 16-wide slices of the head dimension
  constexpr int kRowChunks = D / CH;
  constexpr int kStageFloats = 2 * KT * LD;
  constexpr int kMergeLd = kPrefillQueries + 1;  // merge rows padded: conflict-free dimension-major reads
  // Per-wave stage; after the key loop the same memory holds the merge inputs.
  __shared__ __align__(16) float stage[kPrefillWaves][kStageFloats];
  static_assert(kPrefillWaves * kStageFloats >= kPrefillWaves * (3 * kPrefillQueries + D * kMergeLd), "merge must fit");
  const int R = a.hq / a.hkv;
  const int h = blockIdx.y;
  const int g = h / R;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int q0 = blockIdx.x * kPrefillQueries;
  const int qi = lane % 16, kq = lane / 16;  // query column, k slot
  const int qrow = min(q0 + qi, a.tokens - 1);
  const int qpos = a.start + q0 + qi;
  float* k_s = stage[wave];            // [KT][LD]
  float* v_s = stage[wave] + KT * LD;  // [KT][LD]
  // fp16 cache (d % 32 == 0): K and V stay fp16 in the stage and both
  // products run on the fp16 matrix cores, with q and p split hi + lo.
  constexpr bool kF16 = std::is_same<KV, __half>::value && D % 32 == 0;
  constexpr int LDH = D + 8;  // halves per fp16 stage row: 16-byte aligned, 13 x 16 bytes for d 96
  static_assert(!kF16 || 2 * KT * LDH * 2 <= kStageFloats * 4, "fp16 stage must fit");
  _Float16* kh_s = reinterpret_cast<_Float16*>(stage[wave]);  // [KT][LDH]
  _Float16* vh_s = kh_s + KT * LDH;                            // [KT][LDH]

  const int last_key = a.start + min(q0 + kPrefillQueries, a.tokens) - 1;  // the block's last query position
  const int n_tiles = last_key / KT + 1;
  // chunk c: key c / kRowChunks, dims (c % kRowChunks) * CH ..: consecutive
  // lanes read consecutive 16 bytes of a row.
  // A tile's 16 keys lie in one KV page (pages hold 64 aligned tokens), where
  // one head's rows are contiguous: one segment lookup per tile.
  auto fetch = [&](int tile, Regs& r) {
    const int t0 = tile * KT;
    const int seg = kv_segment(t0);
    const int64_t tile_off = kv_segment_offset(seg, t0, g, a.hkv, D);
    const KV* ktile = static_cast<const KV*>(a.seg.s[seg].k) + tile_off;
    const KV* vtile = static_cast<const KV*>(a.seg.s[seg].v) + tile_off;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = min(lane + i * kWave, kChunks - 1);
      const int key = min(t0 + c / kRowChunks, last_key);  // rows past the last key are masked
      const int64_t off = static_cast<int64_t>(key - t0) * D + (c % kRowChunks) * CH;
      r.k[i] = *reinterpret_cast<const uint4*>(ktile + off);
      r.v[i] = *reinterpret_cast<const uint4*>(vtile + off);
    }
  };
  Regs regs;
  fetch(min(wave, n_tiles - 1), regs);  // unconditional; a wave with no tile never reads it

  // Q^T fragments: dims 16j + 4 kq + {0..3} of query qi (fp32), or dims
  // 32j + 8 kq + {0..7} split into fp16 hi + lo (fp16 path).  q is scaled
  // once by log2(e) / sqrt(d): the scores come out in base-2 units, already
  // divided by sqrt(d) (decoder_layer.cpp:213 divides each score), and the
  // softmax takes exp2 (v_exp_f32) instead of expf.  The two forms differ by
  // rounding only.
  const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(D));
  float4 qf[kF16 ? 1 : DT];
  uint4 qh[kF16 ? D / 32 : 1], ql[kF16 ? D / 32 : 1];  // f16x8 bits
  const float* qsrc = a.query + static_cast<int64_t>(qrow) * a.query_stride + h * D;
  if constexpr (kF16) {
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      const float4 x0 = *reinterpret_cast<const float4*>(qsrc + 32 * j + 8 * kq);
      const float4 x1 = *reinterpret_cast<const float4*>(qsrc + 32 * j + 8 * kq + 4);
      const float x[8] = {x0.x * qscale, x0.y * qscale, x0.z * qscale, x0.w * qscale,
                          x1.x * qscale, x1.y * qscale, x1.z * qscale, x1.w * qscale};
      f16x8 hv, lv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hv[e] = static_cast<_Float16>(x[e]);
        lv[e] = static_cast<_Float16>(x[e] - static_cast<float>(hv[e]));
      }
      qh[j] = __builtin_bit_cast(uint4, hv);
      ql[j] = __builtin_bit_cast(uint4, lv);
    }
  } else {
#pragma unroll
    for (int j = 0; j < DT; ++j) {
      const float4 x = *reinterpret_cast<const float4*>(qsrc + 16 * j + 4 * kq);
      qf[j] = make_float4(x.x * qscale, x.y * qscale, x.z * qscale, x.w * qscale);
    }
  }

  f32x4 ot[DT];  // O^T[d = 16 dt + 4 kq + i][query qi]
#pragma unroll
  for (int j = 0; j < DT; ++j) ot[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY, l_part = 0.0f;

  auto step = [&](int tile, auto prefetch) {
    const int t0 = tile * KT;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = lane + i * kWave;
      if (kF16 && c < kChunks) {
        const int r = c / kRowChunks, col = (c % kRowChunks) * CH;
        // Component-wise (a whole-struct copy would keep regs in scratch).
        const uint4 kc = regs.k[i], vc = regs.v[i];
        *reinterpret_cast<u32x4*>(&kh_s[r * LDH + col]) = u32x4{kc.x, kc.y, kc.z, kc.w};
        *reinterpret_cast<u32x4*>(&vh_s[r * LDH + col]) = u32x4{vc.x, vc.y, vc.z, vc.w};
      } else if (c < kChunks) {
        const int r = c / kRowChunks, col = (c % kRowChunks) * CH;
        float kf[CH], vf[CH];
        chunk_to_float_n<KV>(regs.k[i], kf);
        chunk_to_float_n<KV>(regs.v[i], vf);
#pragma unroll
        for (int e = 0; e < CH; e += 4) {
          *reinterpret_cast<float4*>(&k_s[r * LD + col + e]) = make_float4(kf[e], kf[e + 1], kf[e + 2], kf[e + 3]);
          *reinterpret_cast<float4*>(&v_s[r * LD + col + e]) = make_float4(vf[e], vf[e + 1], vf[e + 2], vf[e + 3]);
        }
      }
    }
    // The registers are free: the wave's next tile loads overlap this tile's
    // work (a compile-time choice; a guarded load would be waited for where the
    // branches join).
    if constexpr (decltype(prefetch)::value) fetch(tile + kPrefillWaves, regs);
    // The stage is private to this wave, and a wave's LDS operations complete
    // in order: waiting for the writes is enough before other lanes read them.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    f32x4 st[KT / 16];
#pragma unroll
    for (int kt = 0; kt < KT / 16; ++kt) {
      st[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (kF16) {
        // A = K (key qi, dims 32j + 8 kq ..), B = Q^T: 32 dims per product.
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
          const f16x8 kf = *reinterpret_cast<const f16x8*>(&kh_s[(kt * 16 + qi) * LDH + 32 * j + 8 * kq]);
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(f16x8, qh[j]), st[kt], 0, 0, 0);
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(f16x8, ql[j]), st[kt], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < DT; ++j) {
          const float4 kf = *reinterpret_cast<const float4*>(&k_s[(kt * 16 + qi) * LD + 16 * j + 4 * kq]);
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.x, qf[j].x, st[kt], 0, 0, 0);
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.y, qf[j].y, st[kt], 0, 0, 0);
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.z, qf[j].z, st[kt], 0, 0, 0);
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.w, qf[j].w, st[kt], 0, 0, 0);
        }
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT / 16; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = t0 + kt * 16 + 4 * kq + i;
        st[kt][i] = key <= qpos ? st[kt][i] : -INFINITY;
        mx = fmaxf(mx, st[kt][i]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    // No key of this query seen yet (m_new = -inf): everything stays zero.
    const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_part *= alpha;
#pragma unroll
    for (int j = 0; j < DT; ++j) ot[j] *= alpha;
#pragma unroll
    for (int kt = 0; kt < KT / 16; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st[kt][i] = st[kt][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st[kt][i] - m_new);
        l_part += st[kt][i];
      }
    m_run = m_new;
    // O^T += V^T P^T over the tile's keys.  fp16 path: one 16x16x16 product
    // per (slice, plane): lane l supplies keys 4 kq + {0..3}, which are the
    // rows of S^T it holds, so p goes in as is (split hi + lo).
    if constexpr (kF16) {
#pragma unroll
      for (int kt = 0; kt < KT / 16; ++kt) {
        f16x4 ph, pl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ph[i] = static_cast<_Float16>(st[kt][i]);
          pl[i] = static_cast<_Float16>(st[kt][i] - static_cast<float>(ph[i]));
        }
#pragma unroll
        for (int j = 0; j < DT; ++j) {
          // A = V^T: lane (qi, kq) needs V[key 4 kq + i][dim 16 j + qi], i = 0..3,
          // a column of the 4 x 16 block of V rows 4 kq .. 4 kq + 3, dims 16 j ..
          // One transposing LDS read (ds_read_b64_tr_b16) delivers it: within a
          // 16-lane group, lane i receives element i % 4 of the 8 bytes that lane
          // 4 k + i / 4 addresses, for k = 0..3; so lane qi addresses row qi / 4,
          // dims 4 (qi % 4) .. + 3 of the block.
          const _Float16* vsrc = &vh_s[(kt * 16 + 4 * kq + qi / 4) * LDH + 16 * j + 4 * (qi % 4)];
          const f16x4 va = __builtin_bit_cast(
              f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(vsrc)));
          ot[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, ot[j], 0, 0, 0);
          ot[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, ot[j], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int kt = 0; kt < KT / 16; ++kt)
#pragma unroll
        for (int j = 0; j < DT; ++j) {
          const float* vcol = &v_s[(kt * 16 + 4 * kq) * LD + 16 * j + qi];
          const float v0 = vcol[0], v1 = vcol[LD], v2 = vcol[2 * LD], v3 = vcol[3 * LD];
          ot[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0, st[kt][0], ot[j], 0, 0, 0);
          ot[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1, st[kt][1], ot[j], 0, 0, 0);
          ot[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(v2, st[kt][2], ot[j], 0, 0, 0);
          ot[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(v3, st[kt][3], ot[j], 0, 0, 0);
        }
    }
    // Reads of this stage finish before the next tile's writes (in-order LDS).
  };
  int tile = wave;
  for (; tile + kPrefillWaves < n_tiles; tile += kPrefillWaves) step(tile, std::true_type{});
  if (tile < n_tiles) step(tile, std::false_type{});

  // ---- merge the four waves: (m, l) per query, O^T fragments ----
  float l = l_part + __shfl_xor(l_part, 16);
  l += __shfl_xor(l, 32);
  __syncthreads();  // every wave is done with its stage
  float* mrg = &stage[0][0];  // [wave][16] m, [wave][16] l, [wave][D][kMergeLd] o
  float* m_sh = mrg;
  float* l_sh = mrg + kPrefillWaves * kPrefillQueries;
  float* o_sh = mrg + 2 * kPrefillWaves * kPrefillQueries;
  if (kq == 0) {
    m_sh[wave * kPrefillQueries + qi] = m_run;
    l_sh[wave * kPrefillQueries + qi] = l;
  }
#pragma unroll
  for (int j = 0; j < DT; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) o_sh[(wave * D + 16 * j + 4 * kq + i) * kMergeLd + qi] = ot[j][i];
  __syncthreads();
  // Per query: the waves' weights e_w = exp(m_w - M) / L (M finite: wave 0
  // holds key 0 of every query), in place of m.
  if (threadIdx.x < kPrefillQueries) {
    const int q = threadIdx.x;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kPrefillWaves; ++w) M = fmaxf(M, m_sh[w * kPrefillQueries + q]);
    float e[kPrefillWaves];
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kPrefillWaves; ++w) {
      const float mw = m_sh[w * kPrefillQueries + q];
      e[w] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      L = fmaf(l_sh[w * kPrefillQueries + q], e[w], L);
    }
    const float inv = 1.0f / L;
#pragma unroll
    for (int w = 0; w < kPrefillWaves; ++w) m_sh[w * kPrefillQueries + q] = e[w] * inv;
  }
  __syncthreads();
  // Every thread runs the same trip count (16 D is a multiple of the block
  // for d % 32 == 0), so the 32-lane chunk reductions below see whole waves.
  for (int idx = threadIdx.x; idx < kPrefillQueries * D; idx += kWave * kPrefillWaves) {
    const int q = idx / D, dim = idx % D;
    const bool valid = q0 + q < a.tokens;
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < kPrefillWaves; ++w) o = fmaf(o_sh[(w * D + dim) * kMergeLd + q], m_sh[w * kPrefillQueries + q], o);
    const int64_t off = static_cast<int64_t>(q0 + q) * a.out_stride + h * D + dim;
    if (a.out && valid) a.out[off] = o;
    if constexpr (D % kSplitChunkFine == 0) {
      if (a.out_split.hi) {
        // 32 consecutive dims of one query per chunk (the lanes of a half wave).
        const float mx = group_max<kSplitChunkFine>(valid ? fabsf(o) : 0.0f);
        int e = 0;
        frexpf(mx, &e);  // e = 0 for a zero chunk
        e = max(e, -100);
        if (valid) {
          const float xs = o * ldexpf(1.0f, 15 - e);
          const _Float16 hh = static_cast<_Float16>(xs);
          const _Float16 ll = static_cast<_Float16>(xs - static_cast<float>(hh));
          __builtin_memcpy(a.out_split.hi + off, &hh, 2);
          __builtin_memcpy(a.out_split.lo + off, &ll, 2);
          if (dim % kSplitChunkFine == 0)
            a.out_split.inv[static_cast<int64_t>(q0 + q) * (a.hq * D / kSplitChunkFine) + (h * D + dim) / kSplitChunkFine] =
                ldexpf(1.0f, e - 15);
        }
      }
    }
  }
}

template <int BM, int BN, int kMode>
void launch_gemm_tile_epi(const GemmArgs& g, hipStream_t s) {
  const dim3 grid((g.n + BN - 1) / BN, (g.m + BM - 1) / BM, g.k_splits);
  if (g.swiglu) {
    gemm_f16w_kernel<BM, BN, kGemmEpiSwiGlu, kMode><<<grid, kGemmThreads, 0, s>>>(g);
  } else if (g.residual) {
    gemm_f16w_kernel<BM, BN, kGemmEpiResidual, kMode><<<grid, kGemmThreads, 0, s>>>(g);
  } else {
    gemm_f16w_kernel<BM, BN, kGemmEpiStore, kMode><<<grid, kGemmThreads, 0, s>>>(g);
  }
}

template <int BM, int BN>
hipError_t launch_gemm_tile(const GemmArgs& g, hipStream_t s) {
  if (!g.a_hi) {
    launch_gemm_tile_epi<BM, BN, kSplitNone>(g, s);
  } else if (g.a_chunk == kSplitChunk) {
    launch_gemm_tile_epi<BM, BN, kSplitTile>(g, s);
  } else {
    // Fine planes feed the split-K partial products (O, down) only.
    const dim3 grid((g.n + BN - 1) / BN, (g.m + BM - 1) / BM, g.k_splits);
    gemm_f16w_kernel<BM, BN, kGemmEpiStore, kSplitFine><<<grid, kGemmThreads, 0, s>>>(g);
  }
  return hipGetLastError();
}

template <int BM, int BN, int kGran>
void launch_gemm_dma_epi(const GemmArgs& g, hipStream_t s) {
  const dim3 grid((g.n + BN - 1) / BN, (g.m + BM - 1) / BM, g.k_splits);
  if (g.swiglu) {
    gemm_dma_kernel<BM, BN, kGemmEpiSwiGlu, kGran><<<grid, kGemmThreads, 0, s>>>(g);
  } else if (g.residual) {
    gemm_dma_kernel<BM, BN, kGemmEpiResidual, kGran><<<grid, kGemmThreads, 0, s>>>(g);
  } else {
    gemm_dma_kernel<BM, BN, kGemmEpiStore, kGran><<<grid, kGemmThreads, 0, s>>>(g);
  }
}

template <int BM, int BN>
hipError_t launch_gemm_dma(const GemmArgs& g, hipStream_t s) {
  if (g.a_chunk == kSplitChunk) {
    launch_gemm_dma_epi<BM, BN, kSplitChunk>(g, s);
  } else {
    launch_gemm_dma_epi<BM, BN, kSplitChunkFine>(g, s);
  }
  return hipGetLastError();
}

// The direct-to-LDS kernel takes pre-split A with K a multiple of its stage.
bool use_gemm_dma(const GemmArgs& g) {
  // Its per-lane load offsets are 32-bit byte offsets from the operands' bases.
  const int64_t a_bytes = static_cast<int64_t>(g.m) * g.lda * 2, w_bytes = static_cast<int64_t>(g.n) * g.k * 2;
  const int64_t s_bytes = static_cast<int64_t>(g.m) * ((g.k + kSplitChunkFine - 1) / kSplitChunkFine) * 4;
  return !g.register_staged && g.a_hi != nullptr && g.k % kDmaBK == 0 && g.lda % 8 == 0 && a_bytes < (int64_t{1} << 32) &&
         w_bytes < (int64_t{1} << 32) && s_bytes < (int64_t{1} << 32);
}

template <int BM, int BN>
hipError_t launch_gemm_any(const GemmArgs& g, hipStream_t s) {
  if (!use_gemm_dma(g)) return launch_gemm_tile<BM, BN>(g, s);
  // The direct-to-LDS kernel runs 64 x 128 tiles as 64 x 64 (more blocks per
  // CU measured faster: gate_up 16.5 -> 13.3 us).
  if constexpr (BN == 128) {
    return launch_gemm_dma<BM, 64>(g, s);
  } else {
    return launch_gemm_dma<BM, BN>(g, s);
  }
}

template <typename KV>
hipError_t launch_qkv_rows_kv(const QkvRowsArgs& a, hipStream_t s) {
  const dim3 grid(a.hq + a.hkv, (a.tokens + kQkvRowsTokens - 1) / kQkvRowsTokens);
  const dim3 block(kWave * kQkvRowsTokens);
  switch (a.d) {
    case 16: qkv_rows_kernel<KV, 16><<<grid, block, 0, s>>>(a); break;
    case 32: qkv_rows_kernel<KV, 32><<<grid, block, 0, s>>>(a); break;
    case 64: qkv_rows_kernel<KV, 64><<<grid, block, 0, s>>>(a); break;
    case 96: qkv_rows_kernel<KV, 96><<<grid, block, 0, s>>>(a); break;
    case 128: qkv_rows_kernel<KV, 128><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename KV>
hipError_t launch_prefill_attention_kv(const PrefillAttnArgs& a, hipStream_t s) {
  const dim3 grid((a.tokens + kPrefillQueries - 1) / kPrefillQueries, a.hq);
  const dim3 block(kWave * kPrefillWaves);
  switch (a.d) {
    case 16: prefill_attention_kernel<KV, 16><<<grid, block, 0, s>>>(a); break;
    case 32: prefill_attention_kernel<KV, 32><<<grid, block, 0, s>>>(a); break;
    case 64: prefill_attention_kernel<KV, 64><<<grid, block, 0, s>>>(a); break;
    case 96: prefill_attention_kernel<KV, 96><<<grid, block, 0, s>>>(a); break;
    case 128: prefill_attention_kernel<KV, 128><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool gemm_supported(int m, int n, int k) { return m > 0 && n > 0 && k > 0 && k % 8 == 0; }

template <int BT>
hipError_t launch_gemm_skinny(const GemmArgs& g, hipStream_t s) {
  const dim3 grid((g.n + 15) / 16);
  if (g.residual) {
    gemm_skinny_kernel<BT, true><<<grid, kWave * kSkinnyWaves, 0, s>>>(g);
  } else {
    gemm_skinny_kernel<BT, false><<<grid, kWave * kSkinnyWaves, 0, s>>>(g);
  }
  return hipGetLastError();
}

namespace {
bool use_skinny(int m, int k) { return m <= 32 && k % 32 == 0 && k >= 32 * kSkinnyWaves; }

// Tiling of a launch_gemm call (tile and K split count); the consumers of the
// split-K partials read the split count from gemm_k_splits.
struct GemmTiling {
  int bm = 32, bn = 32, splits = 1;
};
constexpr int64_t kGemmTargetBlocks = 768;

GemmTiling choose_gemm_tiling(int m, int n, int k) {
  const int nk = (k + kGemmBK - 1) / kGemmBK;
  const int max_splits = std::max(1, std::min(8, nk / 2));
  // Unsplit: 64 x 128 when that gives every CU two blocks, else 64 x 64 when
  // that does (gate_up at M = 512: 512 blocks, 13.3 us on the direct-to-LDS
  // kernel, 16.7 register-staged; 64 x 128 measured 16.5).  Else 32 x 64
  // tiles split along K until the launch reaches kGemmTargetBlocks (the
  // direct-to-LDS kernel with two stages fits four such blocks per CU): at
  // M = 512 down 768 x 2048 10.5 us with 4 splits (64 x 64 with 4: 11.4),
  // QKV 6.3 us with 3, O 5.8-6.3 us with 2-4.
  const int64_t wide = static_cast<int64_t>((m + 63) / 64) * ((n + 127) / 128);
  if (wide >= 512) return {64, 128, 1};
  if (2 * wide >= 512) return {64, 64, 1};
  const int64_t blocks = static_cast<int64_t>((m + 31) / 32) * ((n + 63) / 64);
  const int64_t need = (kGemmTargetBlocks + blocks - 1) / blocks;
  return {32, 64, static_cast<int>(std::min<int64_t>(std::max<int64_t>(need, 1), max_splits))};
}
}  // namespace

int gemm_k_splits(int m, int n, int k) {
  if (!gemm_supported(m, n, k) || use_skinny(m, k)) return 1;
  return choose_gemm_tiling(m, n, k).splits;
}

bool gemm_presplit_supported(int m, int n, int k) { return gemm_supported(m, n, k) && !use_skinny(m, k); }

bool gemm_swiglu_split_supported(int m, int n, int k) {
  const GemmTiling t = choose_gemm_tiling(m, n, k);
  return gemm_swiglu_supported(m, n, k) && n % (2 * kSplitChunkFine) == 0 && (t.bn == 128 || t.bn == 64);
}

bool gemm_swiglu_supported(int m, int n, int k) {
  return gemm_supported(m, n, k) && !use_skinny(m, k) && n % 2 == 0 && choose_gemm_tiling(m, n, k).splits == 1;
}

hipError_t launch_gemm(const GemmArgs& g, hipStream_t s) {
  if (!gemm_supported(g.m, g.n, g.k) || g.lda % 4 != 0 || g.lda < g.k || g.ldc < (g.swiglu ? g.n / 2 : g.n))
    return hipErrorInvalidValue;
  // Pre-split A: all three planes, 16-byte rows, and the tiled path; fine
  // (32-column) scales only for the plain store.
  if (g.a_hi && (!g.a_lo || !g.a_inv || g.lda % 8 != 0 || use_skinny(g.m, g.k) ||
                 (g.a_chunk != kSplitChunk && g.a_chunk != kSplitChunkFine) ||
                 (g.a_chunk == kSplitChunkFine && (g.swiglu || g.residual))))
    return hipErrorInvalidValue;
  if (!g.a_hi && !g.a) return hipErrorInvalidValue;
  // act pre-split: the SwiGLU epilogue on unsplit 64 x 128, 64 x 64 or 32 x 64 tiles, all three planes,
  // 8-byte rows.
  if (g.act_split.hi && (!g.swiglu || !g.act_split.lo || !g.act_split.inv || g.ldc % 4 != 0 ||
                         !gemm_swiglu_split_supported(g.m, g.n, g.k)))
    return hipErrorInvalidValue;
  if (!g.c && !g.act_split.hi) return hipErrorInvalidValue;
  if (g.swiglu && (g.k_splits != 1 || g.residual || !gemm_swiglu_supported(g.m, g.n, g.k)))
    return hipErrorInvalidValue;
  if (g.k_splits < 1 || (g.k_splits > 1 && (g.residual || g.split_stride < static_cast<int64_t>(g.m) * g.ldc ||
                                            g.k_splits > gemm_k_splits(g.m, g.n, g.k))))
    return hipErrorInvalidValue;
  // Few rows (batched decode): stream W with one block per 16 rows of W.
  if (use_skinny(g.m, g.k)) return g.m <= 16 ? launch_gemm_skinny<1>(g, s) : launch_gemm_skinny<2>(g, s);
  // Calls with the chooser's split count take its tile.
  const GemmTiling t = choose_gemm_tiling(g.m, g.n, g.k);
  if (g.k_splits == t.splits) {
    if (t.bn == 128) return launch_gemm_any<64, 128>(g, s);
    if (t.bm == 64) return launch_gemm_any<64, 64>(g, s);
    if (t.bn == 64) return launch_gemm_any<32, 64>(g, s);
    return launch_gemm_any<32, 32>(g, s);
  }
  // Otherwise the largest tile that still gives every CU a block (256 CUs,
  // counting the K splits), else the smallest tile.
  auto blocks = [&](int bm, int bn) {
    return static_cast<int64_t>((g.m + bm - 1) / bm) * ((g.n + bn - 1) / bn) * g.k_splits;
  };
  if (blocks(64, 128) >= 256) return launch_gemm_any<64, 128>(g, s);
  if (blocks(64, 64) >= 256) return launch_gemm_any<64, 64>(g, s);
  if (blocks(32, 64) >= 256) return launch_gemm_any<32, 64>(g, s);
  return launch_gemm_any<32, 32>(g, s);
}

hipError_t launch_qkv_rows(const QkvRowsArgs& a, KvDtype kv, hipStream_t stream) {
  if (!attention_supported(a.hq, a.hkv, a.d) || a.tokens <= 0 || a.qkv_parts < 1 ||
      a.qkv_parts > kQkvRowsMaxParts || (a.qkv_parts > 1 && a.qkv_part_stride < int64_t{a.tokens} * a.qkv_stride))
    return hipErrorInvalidValue;
  return kv == kKvF16 ? launch_qkv_rows_kv<__half>(a, stream) : launch_qkv_rows_kv<float>(a, stream);
}

hipError_t launch_prefill_attention(const PrefillAttnArgs& a, KvDtype kv, hipStream_t stream) {
  if (!attention_supported(a.hq, a.hkv, a.d) || a.tokens <= 0 || a.start < 0) return hipErrorInvalidValue;
  if (!a.out && !a.out_split.hi) return hipErrorInvalidValue;
  if (a.out_split.hi && (!a.out_split.lo || !a.out_split.inv || a.out_split.chunk != kSplitChunkFine ||
                         a.d % kSplitChunkFine != 0))
    return hipErrorInvalidValue;
  return kv == kKvF16 ? launch_prefill_attention_kv<__half>(a, stream)
                      : launch_prefill_attention_kv<float>(a, stream);
}

}  // namespace mmr
