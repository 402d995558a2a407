// Host-side interface between the C ABI (scaled_mm_api.hip) and the per-dtype kernel instantiations
// (scaled_mm_launch.hip, compiled once per combination).
#pragma once

#include <hip/hip_runtime.h>

#include "scaled_mm_kernels.h"

namespace feather {

struct TileQuery {
    int warps_m;
    int warps_n;
    int unroll_k;
    int repeat_m;
    int repeat_n;
    bool prefetch;
};

#define FEATHER_COMBO_CAT_(e, a, o) launch_combo_##e##a##o
#define FEATHER_COMBO_FN(e, a, o) FEATHER_COMBO_CAT_(e, a, o)

// launch_combo_<e5m2><a_bf16><out_bf16>: false if the tile is not instantiated, else enqueues the kernel.
bool launch_combo_000(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_001(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_010(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_011(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_100(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_101(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_110(const TileQuery&, const Params&, hipStream_t);
bool launch_combo_111(const TileQuery&, const Params&, hipStream_t);

}  // namespace feather
