// Runtime compilation of GEMM kernels specialised per problem.
//
// Replaces the reference's deep-jit runtime and its per-call kernel generation
// (csrc/jit/jit.hpp:16-92, csrc/jit_kernels/fp8_gemm.hpp:11-81): dg_gemm with `jit` set
// instantiates gemm_body for the chosen tile with the GEMM type, the K split and the
// `compiled_dims` sizes as compile-time constants, compiles it in-process with hipRTC for
// gfx950 (no compiler subprocess), caches the code object on disk and launches it through
// hipModuleLaunchKernel.
//
// Cache: DG_JIT_CACHE_DIR, a ':'-separated list of directories searched front to back (the
// first hit wins, a miss compiles into the first), default $HOME/.deep_gemm_amd/cache.  The
// key hashes the generated source, the kernel headers' text, the compile options and the
// hipRTC version, so editing a header never reuses a stale code object.  Files are written to
// a temporary name and renamed, so concurrent processes never read a partial file.
#include <hip/hiprtc.h>

#include <dlfcn.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "gemm_tiles.hpp"
#include "../../include/deep_gemm_amd.h"

extern "C" int dg_set_error(const char* msg);

namespace dg {
namespace {

std::mutex g_mu;
std::string g_include_dir;                      // directory holding gemm_kernel.hpp / dg_common.hpp
std::string g_headers[2];                       // their text, read once
bool g_headers_read = false;
std::unordered_map<std::string, std::vector<char>> g_code;             // key -> code object
std::unordered_map<std::string, hipFunction_t> g_fn;                    // key@device -> kernel
int64_t g_stat_compiled = 0, g_stat_disk = 0, g_stat_mem = 0;

const char* const kHeaderNames[2] = {"gemm_kernel.hpp", "dg_common.hpp"};
const char* const kOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++20",
                                // packed fp32 VALU ops stay off, as in the ahead-of-time build
                                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
constexpr int kNumOptions = sizeof(kOptions) / sizeof(kOptions[0]);

uint64_t fnv1a(uint64_t h, const std::string& s) {
    for (unsigned char c : s) h = (h ^ c) * 1099511628211ull;
    return h;
}

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::stringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

// Default header directory: csrc/ next to the library's package directory.
std::string default_include_dir() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&default_include_dir), &info) == 0 || info.dli_fname == nullptr) return "";
    std::string so = info.dli_fname;
    const size_t slash = so.rfind('/');
    const std::string dir = slash == std::string::npos ? "." : so.substr(0, slash);
    return dir + "/../csrc";
}

bool load_headers() {
    if (g_headers_read) return true;
    if (g_include_dir.empty()) g_include_dir = default_include_dir();
    for (int i = 0; i < 2; ++i) {
        if (!read_file(g_include_dir + "/" + kHeaderNames[i], g_headers[i])) {
            const std::string msg = "dg_jit: cannot read " + g_include_dir + "/" + kHeaderNames[i] +
                                    " (set the kernel header directory with dg_jit_set_include_dir)";
            dg_set_error(msg.c_str());
            return false;
        }
    }
    g_headers_read = true;
    return true;
}

std::vector<std::string> cache_dirs() {
    std::vector<std::string> dirs;
    const char* env = std::getenv("DG_JIT_CACHE_DIR");
    std::string list = env && *env ? env : "";
    if (list.empty()) {
        const char* home = std::getenv("HOME");
        list = home && *home ? std::string(home) + "/.deep_gemm_amd/cache"
                             : "/tmp/deep_gemm_amd-" + std::to_string((long)getuid()) + "/cache";
    }
    size_t start = 0;
    while (start <= list.size()) {
        const size_t colon = list.find(':', start);
        const std::string d = list.substr(start, colon == std::string::npos ? std::string::npos : colon - start);
        if (!d.empty()) dirs.push_back(d);
        if (colon == std::string::npos) break;
        start = colon + 1;
    }
    return dirs;
}

void make_dirs(const std::string& path) {
    for (size_t i = 1; i <= path.size(); ++i) {
        if (i == path.size() || path[i] == '/') mkdir(path.substr(0, i).c_str(), 0755);
    }
}

struct Spec {
    TileCfg t;
    int kind, epi, ct, cs, cm, cn, ck;
};

std::string source_of(const Spec& s) {
    char buf[768];
    snprintf(buf, sizeof(buf),
             "#include \"gemm_kernel.hpp\"\n"
             "extern \"C\" __global__ __launch_bounds__(%d, %d) void dg_jit_kernel(const dg::KParams p) {\n"
             "    dg::gemm_body<%d, %d, %d, %d, %d, %d, %d, %d, %d, %d, %d, %d, %d, %d, %d, false, false, %d>(p, blockIdx.x + p.vbase);\n"
             "}\n",
             s.t.nw * 64, s.t.occ * s.t.nw / 4, s.t.bm, s.t.bn, s.t.wgm, s.t.nw, s.t.lw, s.t.stages, s.t.km, s.t.occ,
             s.kind, s.epi, s.ct, s.cs, s.cm, s.cn, s.ck, s.t.nsb);
    return buf;
}

// Code object of `src` (memory, then disk, then hipRTC); `key` receives its cache key.
bool code_object(const std::string& src, std::string& key, const std::vector<char>*& code) {
    uint64_t h = 1469598103934665603ull;
    h = fnv1a(h, src);
    h = fnv1a(h, g_headers[0]);
    h = fnv1a(h, g_headers[1]);
    for (int i = 0; i < kNumOptions; ++i) h = fnv1a(h, kOptions[i]);
    int major = 0, minor = 0;
    hiprtcVersion(&major, &minor);
    h = fnv1a(h, std::to_string(major) + "." + std::to_string(minor));
    char hex[32];
    snprintf(hex, sizeof(hex), "%016llx", (unsigned long long)h);
    key = std::string("dg_gemm_") + hex;

    auto it = g_code.find(key);
    if (it != g_code.end()) {
        code = &it->second;
        return true;
    }
    const std::vector<std::string> dirs = cache_dirs();
    for (const std::string& d : dirs) {
        std::string bytes;
        if (read_file(d + "/" + key + ".hsaco", bytes) && !bytes.empty()) {
            ++g_stat_disk;
            code = &(g_code[key] = std::vector<char>(bytes.begin(), bytes.end()));
            return true;
        }
    }
    hiprtcProgram prog;
    const char* hdr[2] = {g_headers[0].c_str(), g_headers[1].c_str()};
    if (hiprtcCreateProgram(&prog, src.c_str(), "dg_jit_kernel.hip", 2, hdr, kHeaderNames) != HIPRTC_SUCCESS) {
        dg_set_error("dg_jit: hiprtcCreateProgram failed");
        return false;
    }
    const hiprtcResult rc = hiprtcCompileProgram(prog, kNumOptions, kOptions);
    if (rc != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        const std::string msg = std::string("dg_jit: hipRTC compilation failed: ") + hiprtcGetErrorString(rc) + "\n" +
                                log.substr(0, 4000);
        dg_set_error(msg.c_str());
        return false;
    }
    size_t size = 0;
    hiprtcGetCodeSize(prog, &size);
    std::vector<char> bytes(size);
    hiprtcGetCode(prog, bytes.data());
    hiprtcDestroyProgram(&prog);
    ++g_stat_compiled;
    if (!dirs.empty()) {
        make_dirs(dirs[0]);
        const std::string final_path = dirs[0] + "/" + key + ".hsaco";
        const std::string tmp = final_path + ".tmp." + std::to_string((long)getpid());
        std::ofstream f(tmp, std::ios::binary);
        if (f) {
            f.write(bytes.data(), (std::streamsize)bytes.size());
            f.close();
            if (std::rename(tmp.c_str(), final_path.c_str()) != 0) std::remove(tmp.c_str());
        }
    }
    code = &(g_code[key] = std::move(bytes));
    return true;
}

}  // namespace

// Compile (or fetch from the caches) the kernel for one launch plan and, unless compile_only,
// launch it on `st`.
int jit_run(const dg_gemm_args& a, const TileCfg& cfg, int epi, int split, const KParams& p, int64_t grid,
            hipStream_t st, bool compile_only) {
    Spec s;
    s.t = cfg;
    s.kind = a.kind;
    s.epi = epi;
    s.ct = a.gemm_type;
    s.cs = split;
    const int dims = a.compiled_dims;
    s.cm = (dims & DG_COMPILED_M) ? a.m : 0;
    s.cn = (dims & DG_COMPILED_N) ? a.n : 0;
    // (a K-grouped launch contracts a different K per group)
    s.ck = (dims & DG_COMPILED_K) && a.gemm_type != kKGrouped ? a.k : 0;
    const std::string src = source_of(s);
    hipFunction_t fn = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!load_headers()) return DG_EINVAL;
        std::string key;
        const std::vector<char>* code = nullptr;
        if (!code_object(src, key, code)) return DG_ENOKERNEL;
        if (compile_only) return DG_OK;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return dg_set_error("dg_jit: hipGetDevice failed");
        const std::string fkey = key + "@" + std::to_string(dev);
        auto it = g_fn.find(fkey);
        if (it != g_fn.end()) {
            ++g_stat_mem;
            fn = it->second;
        } else {
            hipModule_t mod = nullptr;
            if (hipModuleLoadData(&mod, code->data()) != hipSuccess) return dg_set_error("dg_jit: hipModuleLoadData failed");
            if (hipModuleGetFunction(&fn, mod, "dg_jit_kernel") != hipSuccess)
                return dg_set_error("dg_jit: hipModuleGetFunction failed");
            g_fn.emplace(fkey, fn);   // modules stay loaded for the life of the process
        }
    }
    // (launches of at most `grid` workgroups over the plan's p.vgrid, as for the ahead-of-time kernels)
    for (int base = 0; base < p.vgrid; base += (int)grid) {
        KParams kp = p;
        kp.vbase = base;
        size_t kp_size = sizeof(kp);
        void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &kp, HIP_LAUNCH_PARAM_BUFFER_SIZE, &kp_size, HIP_LAUNCH_PARAM_END};
        const unsigned n = (unsigned)std::min<int64_t>(grid, (int64_t)p.vgrid - base);
        const hipError_t e = hipModuleLaunchKernel(fn, n, 1, 1, (unsigned)(cfg.nw * 64), 1, 1, 0, st, nullptr, config);
        if (e != hipSuccess) {
            dg_set_error(hipGetErrorString(e));
            return DG_ELAUNCH;
        }
    }
    return DG_OK;
}

}  // namespace dg

extern "C" int dg_jit_set_include_dir(const char* dir) {
    if (dir == nullptr || *dir == '\0') return dg_set_error("dg_jit_set_include_dir: empty path");
    std::lock_guard<std::mutex> lk(dg::g_mu);
    dg::g_include_dir = dir;
    dg::g_headers_read = false;
    return DG_OK;
}

extern "C" int dg_jit_stats(int64_t* compiled, int64_t* disk_hits, int64_t* memory_hits) {
    std::lock_guard<std::mutex> lk(dg::g_mu);
    if (compiled) *compiled = dg::g_stat_compiled;
    if (disk_hits) *disk_hits = dg::g_stat_disk;
    if (memory_hits) *memory_hits = dg::g_stat_mem;
    return DG_OK;
}
