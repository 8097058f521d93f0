// prefill_layer.h -- one dense decoder layer over a block of prompt rows.
//
// Counterpart of the reference's run_dense_prefill_layer_device
// (decoder_layer.h:74-80, decoder_layer.cpp:661-734): RMSNorm rows -> fused
// QKV GEMM -> per-head q/k RMSNorm + RoPE + K/V rows into the cache -> causal
// attention -> O GEMM + residual -> RMSNorm rows -> gate_up GEMM + SwiGLU ->
// down GEMM + residual, on the fp16 matrix cores (kernels/prefill.hip), over a
// residual stream updated in place.  The whole-model prefill runs it layer
// after layer on 512-row chunks; the C ABI runs one layer on a caller's rows.
// Nothing here allocates or synchronises: every buffer comes from a
// PrefillScratch carved out of memory the caller owns.
#pragma once

#include "config.h"
#include "device_model.h"
#include "../kernels/kernels.h"

#include <cstddef>
#include <cstdint>

namespace minimind::model {

// Per-call buffers for up to `rows` prompt rows (sizes in prefill_scratch_bytes).
struct PrefillScratch {
  int64_t rows = 0;          // capacity in rows
  float* x = nullptr;        // [rows][H] normalised rows (when the GEMMs read fp32 A)
  mmr::SplitPlanes xs;       // the normalised rows pre-split for the GEMMs
  float* q = nullptr;        // [rows][Hq d] normalised, rotated queries
  float* attn = nullptr;     // [rows][Hq d] attention output
  mmr::SplitPlanes attn_s;   // attention output pre-split
  float* part = nullptr;     // split-K partials of one GEMM
  int64_t part_floats = 0;
  float* act = nullptr;      // [rows][F]
  mmr::SplitPlanes act_s;    // act pre-split
  bool register_staged = false;  // GEMMs on the register-staged kernel only (comparison switch)
};

// Bytes of a scratch for `rows` rows (256-byte aligned slices), and the
// scratch laid out in `base` (which must hold that many bytes).
std::size_t prefill_scratch_bytes(const MiniMindConfig& c, int64_t rows);
PrefillScratch carve_prefill_scratch(const MiniMindConfig& c, int64_t rows, void* base);

// Layer input norm of the first layer: h [rows][H] normalised with `norm`
// into the scratch (the form the QKV GEMM reads for this row count).
void enqueue_prefill_input_norm(const MiniMindConfig& c, const PrefillScratch& s, int rows, const float* h,
                                const float* norm, hipStream_t stream);

// Where one layer's keys and values go and which positions they rotate to.
struct PrefillKv {
  mmr::KvSegs seg;                 // the layer's cache segments
  mmr::KvDtype dtype = mmr::kKvF32;
  int rope_start = 0;              // RoPE position of row 0
  int row0 = 0;                    // cache row of row 0 (rows 0 .. row0 - 1 already cached)
};

// One layer over rows 0 .. rows - 1.  On entry the scratch holds the rows of
// h normalised with the layer's input norm (enqueue_prefill_input_norm, or
// the previous layer's call); h is the residual stream, updated in place.
// Row i's query attends cache rows 0 .. row0 + i.  On exit the scratch holds
// the new h normalised with `next_norm` (the next layer's input norm, or the
// final norm with final_norm set).
void enqueue_prefill_layer(const MiniMindConfig& c, const LayerDev& w, const float* inv_freq, const PrefillScratch& s,
                           const PrefillKv& kv, int rows, float* h, const float* next_norm, bool final_norm,
                           hipStream_t stream);

}  // namespace minimind::model
