// The reference's command-line program (main.cpp, unmodified, where it lies under the reference tree)
// built against this repository's include/ntc_cuda.h with NTC_CUDA=1 and linked against
// libntc_hip.so: the drop-in at link level. On an MI355X, `--cuda` trains on this backend and
// `--cuda-check` runs the reference's own seven-item GPU-vs-CPU harness (main.cpp:2983-3219) against it.
//
// Without NTC_CUDA the same file is the reference's plain CPU program (oracle/_ref/ntc_ref_main,
// target `programs`), which writes the model files and containers the fixtures are made from.
//
// TEST INFRASTRUCTURE ONLY (built into oracle/_ref/ by oracle/Makefile, targets `drop-in` and
// `programs`). As in ref_wrap.cpp, the only addition is the std::fabsf / std::floorf
// using-declarations libstdc++ 11 lacks.
#include <cmath>
namespace std { using ::fabsf; using ::floorf; }
#include "main.cpp"
