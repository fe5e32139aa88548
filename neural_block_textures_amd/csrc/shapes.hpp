// The compile-time MLP shapes the kernels are instantiated for, and the dispatcher that picks
// one for a model (any other model runs through RuntimeShape).
#pragma once
#include "device_common.hpp"

namespace ntc_hip {

//                      C0 C1 C2 pos  H  NL NOUT
using ShapeDefault = FixedShape<4, 0, 0, 1, 24, 2, 3>;    // the reference's default decoder: 64x64x4 latent, uv, 24,24
using Shape256 = FixedShape<4, 0, 0, 1, 16, 2, 3>;        // 256x256 RGB, 64x64x4 bilinear, 16,16
using ShapeTwoLevel = FixedShape<8, 4, 0, 1, 32, 2, 3>;   // 512x512 RGB, 128x128x8 + 32x32x4, 32,32
using ShapeMaterial = FixedShape<2, 4, 0, 1, 32, 2, 12>;  // 4 x 512x512 maps, --qat 2 512x512x2 + 128x128x4, 32,32
using ShapeDct = FixedShape<1, 4, 0, 1, 32, 2, 3>;        // 512x512 RGB, --dct-q 512x512x1 + 128x128x4, 32,32
using ShapeLarge = FixedShape<4, 8, 0, 1, 64, 2, 12>;     // 4 x 2048x2048 maps, 1024x1024x4 + 256x256x8, 64,64

template <class F>
inline const char* dispatch_shape(const DevModel& m, F&& f) {
    if (ShapeMaterial::matches(m)) { f(ShapeMaterial{}); return "2+4|uv|32x2|12"; }
    if (ShapeTwoLevel::matches(m)) { f(ShapeTwoLevel{}); return "8+4|uv|32x2|3"; }
    if (ShapeDct::matches(m)) { f(ShapeDct{}); return "1+4|uv|32x2|3"; }
    if (ShapeLarge::matches(m)) { f(ShapeLarge{}); return "4+8|uv|64x2|12"; }
    if (Shape256::matches(m)) { f(Shape256{}); return "4|uv|16x2|3"; }
    if (ShapeDefault::matches(m)) { f(ShapeDefault{}); return "4|uv|24x2|3"; }
    f(RuntimeShape{});
    return "runtime";
}

}   // namespace ntc_hip
