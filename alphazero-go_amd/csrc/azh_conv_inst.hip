// One compiled instance of the 3x3 convolution: board size AZH_CONV_N and
// workgroup shape kConvTilings[AZH_CONV_TILING], both given on the compiler
// line, or with AZH_RESIDENT_TOWER the board-resident tower of board size
// AZH_CONV_N. The build compiles this file once per instance, so the fully
// unrolled kernels build in parallel.
#include "azh_conv.hpp"

#if !defined(AZH_CONV_N) || (!defined(AZH_CONV_TILING) && !defined(AZH_RESIDENT_TOWER))
#error "AZH_CONV_N and AZH_CONV_TILING (or AZH_RESIDENT_TOWER) must be defined"
#endif

namespace azh {

#if defined(AZH_RESIDENT_TOWER)
template hipError_t launchResidentTowerT<AZH_CONV_N>(const ResidentTower&, int, hipStream_t);
#else
constexpr ConvTiling kInstTiling = kConvTilings[AZH_CONV_TILING];
template hipError_t launchConvT<AZH_CONV_N, kInstTiling.coPerWave, kInstTiling.wavesCo, kInstTiling.wavesPg,
                                kInstTiling.pgPerWave>(const float*, const float*, const float*, const float*,
                                                       const float*, float*, int, int, int, bool, bool,
                                                       hipStream_t);
#endif

} // namespace azh
