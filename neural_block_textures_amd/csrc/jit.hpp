// Kernels specialised at init for a model whose shape is none of the compiled ones (shapes.hpp).
//
// A FixedShape is (level channel counts, positional generators, one hidden width, depth, outputs);
// FixedShapeW the same with a width per hidden layer. A model that shapes.hpp does not list would
// otherwise run on RuntimeShape's kernels, whose per-thread activation arrays live in scratch memory.
// Instead, at init the trainer compiles the shape-templated kernels (kern_valu.hpp, and kern_pop.hpp
// when its hidden layers are one width and the matrix cores pay off) for the model's shape with hipRTC, from the sources next to the library, with the build's own
// compiler options, and launches them from the loaded code object; the result is the same code the
// library holds for its listed shapes. Code objects are cached on disk, keyed by the sources, the
// options and the instantiations (NTC_HIP_JIT_CACHE, else $XDG_CACHE_HOME/ntc_hip or
// ~/.cache/ntc_hip); NTC_HIP_JIT=0 turns the specialisation off.
#pragma once
#include <string>
#include <tuple>
#include <utility>

#include "trainer_impl.hpp"

namespace ntc_hip {

// The model's fixed-shape parameters (level channels, positional generators, outputs, the width of each
// hidden layer); false if the model is outside what the fixed shapes describe.
struct JitShape {
    int C0, C1, C2, npos, NL, nout;
    int H[kMaxHidden];
    bool uniform() const;   // every hidden layer one width: FixedShape (and the matrix kernels may pay off)
};
bool jit_shape_of(const DevModel& m, JitShape& s);
// "ntc_hip::FixedShape<C0, C1, C2, npos, H, NL, nout>", or for unequal widths
// "ntc_hip::FixedShapeW<C0, C1, C2, npos, nout, H0, H1, ...>"
std::string jit_shape_name(const JitShape& s);
// whether the matrix-core kernels pay off for the shape (one hidden width, mfma_pays)
bool jit_shape_mfma(const JitShape& s);

// Compiles (or loads from the cache) the kernels for this trainer's model and makes them current for it
// (I.jit); false, with a reason, when the shape is not one FixedShape describes, hipRTC or the sources
// are missing, or the compiler fails.
bool jit_prepare(Impl& I, std::string& why);
// Compiles the kernel set of the model's shape for arch (e.g. "gfx950") without loading it (no device
// needed); false with the compiler's log as the reason. seconds: the compile time.
bool jit_compile_only(const DevModel& m, const std::string& arch, std::string& why, double* seconds);
// Whether the specialised kernels include the matrix-core ones (the matrix cores pay off for the shape).
bool jit_mfma(const Impl& I);
// The function of one kernel instance: kernel name and the template arguments after the shape.
hipFunction_t jit_function(const Impl& I, const char* kernel, const std::string& targs);

// Launches a specialised kernel with the parameter types of `proto` (the same template instantiated for
// any compiled shape: the parameter list does not depend on the shape), converting the arguments as a
// direct launch would.
template <class... P, class... A>
void jit_launch(void (*proto)(P...), Impl& I, const char* kernel, const std::string& targs, dim3 grid, dim3 block, size_t shm,
                A&&... args) {
    (void)proto;
    std::tuple<std::decay_t<P>...> vals{ std::forward<A>(args)... };
    void* ptrs[sizeof...(P) > 0 ? sizeof...(P) : 1];
    std::apply([&](auto&... v) {
        int i = 0;
        ((ptrs[i++] = (void*)&v), ...);
    }, vals);
    if (I.ext_a) {   // inside a one-launch ProfScope (launch_timed): the dispatch records its events; sizes in work-items
        NTC_CHECK(hipExtModuleLaunchKernel(jit_function(I, kernel, targs), grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x,
                                           block.y, block.z, shm, I.stream, ptrs, nullptr, I.ext_a, I.ext_b, 0));
        I.ext_a = I.ext_b = nullptr;
        return;
    }
    NTC_CHECK(hipModuleLaunchKernel(jit_function(I, kernel, targs), grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)shm,
                                    I.stream, ptrs, nullptr));
}

}   // namespace ntc_hip
