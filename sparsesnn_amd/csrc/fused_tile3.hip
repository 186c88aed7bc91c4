// Instantiations of the tile kernel (tile_kernel.h) for 3x3 / stride 1 / pad 1 convolutions.
#include "tile_kernel.h"
#include "tile3ps.h"

namespace sengine {

// shape: 0 = 8x8 tiles (8-row blocks), 1 = 14x4 (8-row blocks), 2 = 7x7 (7-row blocks).
// pf: prefetch depth (1, or 2 for grids of at most two workgroups per CU; T = 4, one
// channel group per wave).
hipError_t launch_tile3(const TileParams& p, int T, int shape, int gpw, int ksplit, int pf, int oe, int mode,
                        hipStream_t s) {
  switch (T) {
    case 1:
      return launch_tile<1, 3, 8, 8, 8, 1>(p, oe, mode, s);
    case 2:
      return launch_tile<2, 3, 8, 8, 8, 1>(p, oe, mode, s);
    case 4:
      if (ksplit == 2) {
        if (shape == 1) return launch_tile<4, 3, 14, 4, 8, 1, 2>(p, oe, mode, s);
        if (shape == 2)
          return pf == 2 ? launch_tile<4, 3, 7, 7, 7, 1, 2, 2>(p, oe, mode, s)
                         : launch_tile<4, 3, 7, 7, 7, 1, 2>(p, oe, mode, s);
        return launch_tile<4, 3, 8, 8, 8, 1, 2>(p, oe, mode, s);
      }
      if (shape == 1) {
        if (gpw == 2) return launch_tile<4, 3, 14, 4, 8, 2>(p, oe, mode, s);
        return pf == 2 ? launch_tile<4, 3, 14, 4, 8, 1, 1, 2>(p, oe, mode, s)
                       : launch_tile<4, 3, 14, 4, 8, 1>(p, oe, mode, s);
      }
      if (shape == 2) {
        if (gpw == 2) return launch_tile<4, 3, 7, 7, 7, 2>(p, oe, mode, s);
        return pf == 2 ? launch_tile<4, 3, 7, 7, 7, 1, 1, 2>(p, oe, mode, s)
                       : launch_tile<4, 3, 7, 7, 7, 1>(p, oe, mode, s);
      }
      if (gpw == 2) return launch_tile<4, 3, 8, 8, 8, 2>(p, oe, mode, s);
      return pf == 2 ? launch_tile<4, 3, 8, 8, 8, 1, 1, 2>(p, oe, mode, s) : launch_tile<4, 3, 8, 8, 8, 1>(p, oe, mode, s);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_tile3_persistent(const TileParams& p, int shape, int mode, int slots, hipStream_t s) {
  if (shape == 1) return launch_tile3ps<14, 4, 8>(p, mode, slots, s);
  if (shape == 2) return launch_tile3ps<7, 7, 7>(p, mode, slots, s);
  return launch_tile3ps<8, 8, 8>(p, mode, slots, s);
}

hipError_t launch_tile3_persistent_pair(const TileParams& p, int shape, int mode, int slots, hipStream_t s) {
  if (shape == 1) return launch_tile3ps<14, 4, 8, true>(p, mode, slots, s);
  if (shape == 2) return launch_tile3ps<7, 7, 7, true>(p, mode, slots, s);
  return launch_tile3ps<8, 8, 8, true>(p, mode, slots, s);
}

hipError_t launch_tile3_f16in(const TileParams& p, int shape, int ksplit, int out_enc, int mode, hipStream_t s) {
  if (ksplit == 2) {
    if (shape == 1) return launch_tile_f16in<3, 14, 4, 8, 1, 2>(p, out_enc, mode, s);
    if (shape == 2) return launch_tile_f16in<3, 7, 7, 7, 1, 2>(p, out_enc, mode, s);
    return launch_tile_f16in<3, 8, 8, 8, 1, 2>(p, out_enc, mode, s);
  }
  if (shape == 1) return launch_tile_f16in<3, 14, 4, 8>(p, out_enc, mode, s);
  if (shape == 2) return launch_tile_f16in<3, 7, 7, 7>(p, out_enc, mode, s);
  return launch_tile_f16in<3, 8, 8, 8>(p, out_enc, mode, s);
}

}  // namespace sengine
