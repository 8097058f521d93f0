// gemv.hip -- launch planning and dispatch for the GEMV family (kernels in
// gemv_impl.h, instantiated per lane width in gemv_g16/g32/g64.hip).
#include "gemv_impl.h"

namespace mmr {
namespace {

int round_cpl(int needed) {
  static const int kAllowed[] = {1, 2, 3, 4, 6, 8};
  for (int c : kAllowed)
    if (c >= needed) return c;
  return -1;
}

}  // namespace

bool gemv_plan(int rows, int k, GemvEpilogue epi, int lanes_per_row, int rows_per_group, GemvPlan* plan) {
  if (rows <= 0 || k <= 0 || k % 8 != 0) return false;
  const int kchunks = k / 8;
  int g = lanes_per_row;
  if (g == 0) g = kchunks >= 192 ? 64 : (kchunks >= 48 ? 32 : 16);
  if (g != 16 && g != 32 && g != 64) return false;
  int rpg = rows_per_group;
  if (rpg == 0) rpg = (epi == kEpiSwiGlu) ? 2 : 1;
  if (rpg != 1 && rpg != 2 && rpg != 4) return false;
  if (epi == kEpiSwiGlu && (rpg % 2 != 0 || rows % 2 != 0)) return false;
  const int cpl = round_cpl((kchunks + g - 1) / g);
  if (cpl < 0) return false;
  const int rows_per_block = (kGemvBlock / g) * rpg;
  plan->lanes_per_row = g;
  plan->rows_per_group = rpg;
  plan->chunks_per_lane = cpl;
  plan->blocks = (rows + rows_per_block - 1) / rows_per_block;
  return true;
}

hipError_t launch_gemv(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, const GemvPlan& p,
                       hipStream_t stream) {
  const int cpl = p.chunks_per_lane;
#define MMR_GEMV_G(GV, RV)                                               \
  if (p.lanes_per_row == GV && p.rows_per_group == RV)                   \
    return launch_cpl<GV, RV>(a, pro, epi, cpl, p.blocks, stream);
  MMR_GEMV_G(16, 1)
  MMR_GEMV_G(16, 2)
  MMR_GEMV_G(16, 4)
  MMR_GEMV_G(32, 1)
  MMR_GEMV_G(32, 2)
  MMR_GEMV_G(32, 4)
  MMR_GEMV_G(64, 1)
  MMR_GEMV_G(64, 2)
  MMR_GEMV_G(64, 4)
#undef MMR_GEMV_G
  return hipErrorInvalidValue;
}

}  // namespace mmr
