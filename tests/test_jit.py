"""Kernels specialised at init for a model shape the library does not list (csrc/jit.cpp): hipRTC compiles
the shape-templated kernels from the sources next to the library with the build's options. Compiling
needs no device, so the CPU suite checks that both kernel groups compile for new shapes."""
import pytest

from neural_block_textures_amd.trainer import PK_LV1LOCAL, Layout, Trainer


@pytest.mark.parametrize("layout", [
    # 6-7-7-3: the matrix cores would do 36% useful work, so only the VALU kernels are specialised
    Layout(64, 48, [(16, 12, 4, False)], [7, 7], leak=0.01),
    # 6-20-20-3 (58%, the output layer on the VALU)
    Layout(64, 48, [(16, 12, 4, False)], [20, 20], leak=0.01),
    # 6-13-13-3: one partial hidden tile, the population kernel's pixel-per-lane output layer
    Layout(64, 48, [(16, 12, 4, False)], [13, 13], leak=0.01),
    # 8-28-28-12 with --qat and lv1local: the matrix-core kernels too (84% useful)
    Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, False)], [28, 28], T=4, pos=[PK_LV1LOCAL], leak=0.0),
    # 3 levels, clamp output, a leak outside [0, 1] (the selector search's general activation)
    Layout(40, 40, [(40, 40, 1, True), (10, 10, 3, False), (5, 5, 2, False)], [40, 40, 40], leak=1.5, clamp_out=True),
    # hidden layers of different widths (FixedShapeW, VALU kernels only): 20,12 and a deeper 32,16,8
    Layout(32, 32, [(8, 8, 4, False)], [20, 12]),
    Layout(48, 40, [(48, 40, 2, True), (12, 10, 4, False)], [32, 16, 8], T=4, pos=[PK_LV1LOCAL], leak=0.01),
], ids=["valu_7", "mfma_20", "mfma_own_13", "mfma_28", "three_levels", "widths_20_12", "widths_32_16_8"])
def test_specialised_kernels_compile(layout):
    sec, why = Trainer.jit_compile_check(Trainer.model_desc(layout))
    assert sec is not None, why
    assert sec < 120


def test_outside_the_fixed_shapes_is_not_specialised():
    # a hidden layer wider than the envelope's 64 units
    sec, why = Trainer.jit_compile_check(Trainer.model_desc(Layout(32, 32, [(8, 8, 4, False)], [80, 12])))
    assert sec is None and "outside the fixed shapes" in why
