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
// the shapes of the reference's published runs (README.md:690-712; out_m1234/model.bin)
using ShapeM1234 = FixedShape<4, 4, 0, 1, 36, 2, 12>;     // 4 maps, 128x128x4 + 64x64x4, 36,36 (10-36-36-12)
using ShapeDct17 = FixedShape<1, 4, 0, 1, 17, 2, 3>;      // 1-channel DCT plane + 4 channels, 17,17 (7-17-17-3)
using ShapeDct2x17 = FixedShape<2, 4, 0, 1, 17, 2, 3>;    // 2-channel DCT plane + 4 channels, 17,17 (8-17-17-3)
using ShapeDct11 = FixedShape<1, 4, 0, 1, 11, 2, 3>;      // 7-11-11-3
using ShapeDct7 = FixedShape<1, 4, 0, 1, 7, 2, 3>;        // 7-7-7-3
// the reference's published GPU training runs (README.md:358, 382, 531, 956, 1119): selector planes
// with --qat, a nearest block latent, --pos lv1local, 36,36 or 27,27
using ShapeChief1 = FixedShape<1, 2, 0, 1, 36, 2, 3>;     // chief1 --qat 2, 512x512x1 + 128x128x2 (5-36-36-3)
using ShapeMatQat = FixedShape<2, 4, 0, 1, 36, 2, 12>;    // 4 maps --qat 2, 512x512x2 + 128x128x4 (8-36-36-12)
using ShapeChief31 = FixedShape<2, 4, 0, 1, 36, 2, 3>;    // chief1 --qat 3,1, 512x512x2 + 128x128x4 (8-36-36-3)
using ShapeMat3x2 = FixedShape<3, 4, 0, 1, 36, 2, 12>;    // 4 maps, three 2-bit selector channels (9-36-36-12)
using ShapeImage3 = FixedShape<1, 4, 0, 1, 27, 2, 3>;     // --block 8 --qat 4 --qes 8, 27,27 (7-27-27-3)
// the other command lines of the reference's README (README.md:274, 298, 990, 991, 1121, 1123)
using ShapeQat1x4 = FixedShape<1, 4, 0, 1, 36, 2, 3>;     // --qat 2 plane + 4-channel block latent, 36,36 (7-36-36-3)
using ShapeMatQat1x4 = FixedShape<1, 4, 0, 1, 36, 2, 12>; // the same for the 4-texture material (7-36-36-12)
using ShapeRun8 = FixedShape<8, 0, 0, 1, 24, 2, 3>;       // --latent 128 128 8, default 24,24 (10-24-24-3)
using ShapeRun8x3 = FixedShape<8, 4, 0, 1, 24, 2, 9>;     // 3 textures, --latent 128 128 8 --latent2 64 64 4 (14-24-24-9)
using ShapeQes17 = FixedShape<4, 4, 0, 1, 17, 2, 3>;      // --qes 6,8 on two bilinear levels, 17,17 (10-17-17-3)
using ShapeDct2x27 = FixedShape<2, 4, 0, 1, 27, 2, 3>;    // two DCT-coded channels, 27,27 (8-27-27-3)

template <class F>
inline const char* dispatch_shape(const DevModel& m, F&& f) {
    if (ShapeMaterial::matches(m)) { f(ShapeMaterial{}); return "2+4|uv|32x2|12"; }
    if (ShapeTwoLevel::matches(m)) { f(ShapeTwoLevel{}); return "8+4|uv|32x2|3"; }
    if (ShapeDct::matches(m)) { f(ShapeDct{}); return "1+4|uv|32x2|3"; }
    if (ShapeLarge::matches(m)) { f(ShapeLarge{}); return "4+8|uv|64x2|12"; }
    if (Shape256::matches(m)) { f(Shape256{}); return "4|uv|16x2|3"; }
    if (ShapeDefault::matches(m)) { f(ShapeDefault{}); return "4|uv|24x2|3"; }
    if (ShapeM1234::matches(m)) { f(ShapeM1234{}); return "4+4|uv|36x2|12"; }
    if (ShapeDct17::matches(m)) { f(ShapeDct17{}); return "1+4|uv|17x2|3"; }
    if (ShapeDct2x17::matches(m)) { f(ShapeDct2x17{}); return "2+4|uv|17x2|3"; }
    if (ShapeDct11::matches(m)) { f(ShapeDct11{}); return "1+4|uv|11x2|3"; }
    if (ShapeDct7::matches(m)) { f(ShapeDct7{}); return "1+4|uv|7x2|3"; }
    if (ShapeChief1::matches(m)) { f(ShapeChief1{}); return "1+2|uv|36x2|3"; }
    if (ShapeMatQat::matches(m)) { f(ShapeMatQat{}); return "2+4|uv|36x2|12"; }
    if (ShapeChief31::matches(m)) { f(ShapeChief31{}); return "2+4|uv|36x2|3"; }
    if (ShapeMat3x2::matches(m)) { f(ShapeMat3x2{}); return "3+4|uv|36x2|12"; }
    if (ShapeImage3::matches(m)) { f(ShapeImage3{}); return "1+4|uv|27x2|3"; }
    if (ShapeQat1x4::matches(m)) { f(ShapeQat1x4{}); return "1+4|uv|36x2|3"; }
    if (ShapeMatQat1x4::matches(m)) { f(ShapeMatQat1x4{}); return "1+4|uv|36x2|12"; }
    if (ShapeRun8::matches(m)) { f(ShapeRun8{}); return "8|uv|24x2|3"; }
    if (ShapeRun8x3::matches(m)) { f(ShapeRun8x3{}); return "8+4|uv|24x2|9"; }
    if (ShapeQes17::matches(m)) { f(ShapeQes17{}); return "4+4|uv|17x2|3"; }
    if (ShapeDct2x27::matches(m)) { f(ShapeDct2x27{}); return "2+4|uv|27x2|3"; }
    f(RuntimeShape{});
    return "runtime";
}

}   // namespace ntc_hip
