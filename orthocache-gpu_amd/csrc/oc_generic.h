// Portable scoring and decode for the shapes the tuned kernels do not take
// (oc_generic.hip): every power-of-two head_dim up to 512 and tile size up
// to 256 tokens.
#pragma once

#include <hip/hip_runtime.h>

namespace oc {

struct DecodeArgs;

// true when (head_dim, tile_size) is not one of the tuned kernels' shapes
// (head_dim 64 or 128 with 64-token tiles)
bool generic_shape(int head_dim, int tile_size);
// true when the portable kernels take (head_dim, tile_size)
bool generic_supported(int head_dim, int tile_size);
// per-(row, tile) band energies / zeta / keep, or the full transform (o_fwht)
hipError_t gen_launch_score(int dtype, const DecodeArgs& a, int head_dim, hipStream_t st);
// the gated decode into the split partials (a.pm, a.pl, a.pacc; Pg groups)
hipError_t gen_launch_decode(int dtype, const DecodeArgs& a, int head_dim, int gt, int gchunks, hipStream_t st);

}  // namespace oc
