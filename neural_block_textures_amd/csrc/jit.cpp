// Kernels specialised at init for a model whose shape is none of the compiled ones: hipRTC over the
// device-only kernel headers, code objects cached on disk, one loaded module per (device, shape).
#include "jit.hpp"

#include <dlfcn.h>
#include <hip/hiprtc.h>
#include <stdlib.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <vector>

#include "mfma_mlp.hpp"

namespace ntc_hip {

struct JitModuleSet {
    std::string shape;                           // "ntc_hip::FixedShape<...>"
    bool mfma = false;
    std::map<std::string, hipFunction_t> fn;     // name expression -> function
};

namespace {

std::mutex g_mu;
std::map<std::string, JitModuleSet*> g_sets;    // "device|cache key" -> loaded set (kept until the process ends)

// The compiler options of the library's own build (build.py) for the two groups of kernels: every
// fused multiply-add written out, no packed FP32, matrix results straight into VGPRs; the matrix-core
// kernels also with relaxed NaN handling and the IEEE mode bit off.
std::vector<std::string> options(const std::string& arch, const std::string& csrc, bool pop) {
    std::vector<std::string> o = { "--offload-arch=" + arch, "-O3", "-std=c++17", "-ffp-contract=off", "-I" + csrc,
                                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form" };
    if (pop) { o.push_back("-fno-honor-nans"); o.push_back("-mno-amdgpu-ieee"); }
    return o;
}

uint64_t fnv1a(const std::string& s, uint64_t h = 0xcbf29ce484222325ull) {
    for (unsigned char c : s) { h ^= c; h *= 0x100000001b3ull; }
    return h;
}

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

// the directory of this library's sources: csrc/ next to libntc_hip.so
std::string source_dir() {
    Dl_info info{};
    if (!dladdr((void*)&jit_prepare, &info) || !info.dli_fname) return "";
    std::string lib = info.dli_fname;
    const size_t slash = lib.rfind('/');
    return (slash == std::string::npos ? std::string(".") : lib.substr(0, slash)) + "/csrc";
}

std::string cache_dir() {
    if (const char* d = getenv("NTC_HIP_JIT_CACHE")) return d;
    if (const char* x = getenv("XDG_CACHE_HOME")) return std::string(x) + "/ntc_hip";
    if (const char* h = getenv("HOME")) return std::string(h) + "/.cache/ntc_hip";
    return "";
}

void make_dirs(const std::string& path) {
    for (size_t i = 1; i <= path.size(); i++)
        if (i == path.size() || path[i] == '/') mkdir(path.substr(0, i).c_str(), 0755);
}

// the name expressions one program instantiates; pop: the matrix-core kernels, else the VALU ones
std::vector<std::string> expressions(const std::string& shape, const DevModel& m, bool pop) {
    auto e = [&](const char* k, const std::string& t) { return std::string("ntc_hip::") + k + "<" + shape + (t.empty() ? "" : ", " + t) + ">"; };
    std::vector<std::string> v;
    if (!pop) {
        for (const char* k : { "k_batch", "k_pop_eval", "k_decode", "k_lat_pair", "k_qat_search", "k_dct_probe" }) v.push_back(e(k, ""));
        return v;
    }
    const std::string c = m.clamp_out ? "true" : "false";
    const bool unit = m.leak >= 0.0f && m.leak <= 1.0f;
    if (unit) {
        const int a_fd = kActMax, a_es = kActFold;
        v.push_back(e("k_pop_mfma", std::to_string(a_fd) + ", " + c + ", 0"));
        v.push_back(e("k_pop_mfma", std::to_string(a_es) + ", " + c + ", 1"));
        v.push_back(e("k_pop_mfma", std::to_string(a_es) + ", " + c + ", 2"));
        v.push_back(e("k_lat_pair_mfma", std::to_string(a_es) + ", " + c));
    }
    v.push_back(e("k_qat_mfma", std::to_string(unit ? kActFold : kActAny) + ", " + c));
    return v;
}

// one program: compile (or load the cached code object) and return the code and the lowered names
bool build_program(const std::string& csrc, const std::string& arch, const std::string& header, const std::vector<std::string>& exprs,
                   bool pop, const std::string& key_src, std::string& code, std::vector<std::string>& lowered, std::string& why,
                   bool use_cache = true) {
    const auto opts = options(arch, csrc, pop);
    std::string key = key_src + "|" + header + "|" + arch;
    for (const auto& o : opts) key += "|" + o;
    for (const auto& x : exprs) key += "|" + x;
    char hex[17];
    snprintf(hex, sizeof(hex), "%016llx", (unsigned long long)fnv1a(key));
    const std::string dir = use_cache ? cache_dir() : "";
    const std::string base = dir.empty() ? "" : dir + "/ntc_hip_" + hex;
    if (!base.empty()) {
        std::string names;
        if (read_file(base + ".co", code) && read_file(base + ".names", names)) {
            std::istringstream ns(names);
            std::string line;
            lowered.clear();
            while (std::getline(ns, line)) lowered.push_back(line);
            if (lowered.size() == exprs.size() && !code.empty()) return true;
        }
    }
    const std::string src = "#include \"" + header + "\"\n";
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, src.c_str(), "ntc_hip_jit.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
        why = "hiprtcCreateProgram failed"; return false;
    }
    for (const auto& x : exprs) hiprtcAddNameExpression(prog, x.c_str());
    std::vector<const char*> o;
    for (const auto& s : opts) o.push_back(s.c_str());
    const hiprtcResult r = hiprtcCompileProgram(prog, (int)o.size(), o.data());
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        why = "hipRTC could not compile " + header + ": " + log.substr(0, 2000);
        hiprtcDestroyProgram(&prog);
        return false;
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    code.assign(n, '\0');
    hiprtcGetCode(prog, &code[0]);
    lowered.clear();
    for (const auto& x : exprs) {
        const char* l = nullptr;
        if (hiprtcGetLoweredName(prog, x.c_str(), &l) != HIPRTC_SUCCESS || !l) {
            why = "hipRTC has no lowered name for " + x;
            hiprtcDestroyProgram(&prog);
            return false;
        }
        lowered.push_back(l);
    }
    hiprtcDestroyProgram(&prog);
    if (!base.empty()) {   // best effort: a cache that cannot be written only costs the next init a compile
        make_dirs(dir);
        const std::string tmp = base + ".tmp" + std::to_string((long)getpid());
        std::ofstream(tmp + ".co", std::ios::binary).write(code.data(), (std::streamsize)code.size());
        std::string names;
        for (const auto& l : lowered) names += l + "\n";
        std::ofstream(tmp + ".names", std::ios::binary) << names;
        rename((tmp + ".names").c_str(), (base + ".names").c_str());
        rename((tmp + ".co").c_str(), (base + ".co").c_str());
    }
    return true;
}

}   // namespace

bool JitShape::uniform() const {
    for (int l = 1; l < NL; l++) if (H[l] != H[0]) return false;
    return true;
}

bool jit_shape_of(const DevModel& m, JitShape& s) {
    if (m.nlev < 1 || m.nlev > 3 || m.nl < 1 || m.nl > kMaxHidden) return false;
    s.C0 = m.lv[0].C; s.C1 = m.nlev > 1 ? m.lv[1].C : 0; s.C2 = m.nlev > 2 ? m.lv[2].C : 0;
    s.npos = m.npos; s.NL = m.nl; s.nout = m.nout;
    for (int l = 0; l < m.nl; l++) {
        s.H[l] = m.hidden[l];
        if (s.H[l] < 1 || s.H[l] > kMaxWidth) return false;
    }
    // a level of zero channels would read as "no level" in the fixed shapes
    return s.C0 > 0 && (m.nlev < 2 || s.C1 > 0) && (m.nlev < 3 || s.C2 > 0) && s.nout >= 1;
}

std::string jit_shape_name(const JitShape& s) {
    char b[64];
    std::string n;
    if (s.uniform()) {
        snprintf(b, sizeof(b), "ntc_hip::FixedShape<%d, %d, %d, %d, %d, %d, %d>", s.C0, s.C1, s.C2, s.npos, s.H[0], s.NL, s.nout);
        return b;
    }
    snprintf(b, sizeof(b), "ntc_hip::FixedShapeW<%d, %d, %d, %d, %d", s.C0, s.C1, s.C2, s.npos, s.nout);
    n = b;
    for (int l = 0; l < s.NL; l++) n += ", " + std::to_string(s.H[l]);
    return n + ">";
}

bool jit_shape_mfma(const JitShape& s) {
    return s.uniform() && mfma_pays(s.C0 + s.C1 + s.C2 + 2 * s.npos, s.H[0], s.NL, s.nout);
}

bool jit_prepare(Impl& I, std::string& why) {
    if (const char* e = getenv("NTC_HIP_JIT"); e && e[0] == '0') { why = "NTC_HIP_JIT=0"; return false; }
    JitShape js;
    if (!jit_shape_of(I.dm, js)) { why = "the model is outside the fixed shapes"; return false; }
    const std::string shape = jit_shape_name(js);
    const std::string csrc = source_dir();
    std::string key_src;
    for (const char* f : { "kern_pop.hpp", "kern_valu.hpp", "mfma_mlp.hpp", "device_common.hpp", "noise_math.hpp" }) {
        std::string t;
        if (csrc.empty() || !read_file(csrc + "/" + f, t)) { why = "the kernel sources are not next to the library (" + csrc + ")"; return false; }
        key_src += t;
    }
    int rv_major = 0, rv_minor = 0;
    hiprtcVersion(&rv_major, &rv_minor);
    key_src += "|hiprtc " + std::to_string(rv_major) + "." + std::to_string(rv_minor);
    const std::string arch = I.arch.substr(0, I.arch.find(':'));
    const bool mfma = jit_shape_mfma(js);
    const std::string setkey = std::to_string(I.device) + "|" + shape + "|" + std::to_string(I.dm.leak) + "|" + std::to_string(I.dm.clamp_out) +
                               "|" + std::to_string(fnv1a(key_src));
    std::lock_guard<std::mutex> lock(g_mu);
    if (auto it = g_sets.find(setkey); it != g_sets.end()) { I.jit = it->second; return true; }
    auto* set = new JitModuleSet();
    set->shape = shape;
    set->mfma = mfma;
    for (int pop = 0; pop < (mfma ? 2 : 1); pop++) {
        const auto exprs = expressions(shape, I.dm, pop != 0);
        std::string code;
        std::vector<std::string> lowered;
        if (!build_program(csrc, arch, pop ? "kern_pop.hpp" : "kern_valu.hpp", exprs, pop != 0, key_src, code, lowered, why)) {
            delete set;
            return false;
        }
        hipModule_t mod = nullptr;
        if (hipModuleLoadData(&mod, code.data()) != hipSuccess) { why = "hipModuleLoadData failed"; delete set; return false; }
        for (size_t i = 0; i < exprs.size(); i++) {
            hipFunction_t f = nullptr;
            if (hipModuleGetFunction(&f, mod, lowered[i].c_str()) != hipSuccess) { why = "no function " + lowered[i]; delete set; return false; }
            set->fn[exprs[i]] = f;
        }
    }
    g_sets[setkey] = set;
    I.jit = set;
    return true;
}

bool jit_mfma(const Impl& I) { return I.jit && I.jit->mfma; }

bool jit_compile_only(const DevModel& m, const std::string& arch, std::string& why, double* seconds) {
    JitShape js;
    if (!jit_shape_of(m, js)) { why = "the model is outside the fixed shapes"; return false; }
    const std::string shape = jit_shape_name(js), csrc = source_dir();
    const bool mfma = jit_shape_mfma(js);
    const auto t0 = std::chrono::steady_clock::now();
    for (int pop = 0; pop < (mfma ? 2 : 1); pop++) {
        std::string code;
        std::vector<std::string> lowered;
        if (!build_program(csrc, arch, pop ? "kern_pop.hpp" : "kern_valu.hpp", expressions(shape, m, pop != 0), pop != 0, "", code, lowered,
                           why, false))   // compiled every time, never cached
            return false;
        if (code.empty()) { why = "empty code object"; return false; }
    }
    if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return true;
}

hipFunction_t jit_function(const Impl& I, const char* kernel, const std::string& targs) {
    const std::string x = std::string("ntc_hip::") + kernel + "<" + I.jit->shape + (targs.empty() ? "" : ", " + targs) + ">";
    auto it = I.jit->fn.find(x);
    if (it == I.jit->fn.end()) {
        fprintf(stderr, "ntc_hip backend: the kernels specialised for this model hold no %s\n", x.c_str());
        exit(1);
    }
    return it->second;
}

}   // namespace ntc_hip
