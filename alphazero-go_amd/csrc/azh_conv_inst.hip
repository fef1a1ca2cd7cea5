// One compiled instance of the 3x3 convolution: board size AZH_CONV_N and
// workgroup shape kConvTilings[AZH_CONV_TILING], both given on the compiler
// line. The build compiles this file once per (board size, shape), so the
// fully unrolled kernels build in parallel.
#include "azh_conv.hpp"

#if !defined(AZH_CONV_N) || !defined(AZH_CONV_TILING)
#error "AZH_CONV_N and AZH_CONV_TILING must be defined"
#endif

namespace azh {

constexpr ConvTiling kInstTiling = kConvTilings[AZH_CONV_TILING];
template hipError_t launchConvT<AZH_CONV_N, kInstTiling.coPerWave, kInstTiling.wavesCo, kInstTiling.wavesPg,
                                kInstTiling.pgPerWave>(const float*, const float*, const float*, const float*,
                                                       const float*, float*, int, int, int, bool, bool,
                                                       hipStream_t);

} // namespace azh
