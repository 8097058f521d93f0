// gemv_g64.hip -- GEMV instantiations with 64 lanes per row (see gemv_impl.h).
#include "gemv_impl.h"

namespace mmr {

template <int G, int RPG>
hipError_t launch_cpl(const GemvArgs& a, GemvPrologue pro, GemvEpilogue epi, int cpl, int blocks, hipStream_t s) {
  return gemv_detail::launch_cpl_impl<G, RPG>(a, pro, epi, cpl, blocks, s);
}

template hipError_t launch_cpl<64, 1>(const GemvArgs&, GemvPrologue, GemvEpilogue, int, int, hipStream_t);
template hipError_t launch_cpl<64, 2>(const GemvArgs&, GemvPrologue, GemvEpilogue, int, int, hipStream_t);
template hipError_t launch_cpl<64, 4>(const GemvArgs&, GemvPrologue, GemvEpilogue, int, int, hipStream_t);

}  // namespace mmr
