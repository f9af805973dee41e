// libmace_hip.so — host runtime behind include/mace_hip.h.
//
// hipRTC compiles per-layer generated HIP source into a gfx950 code object; the code object is loaded as a
// hipModule on the current device; kernels are launched with hipModuleLaunchKernel on the caller's stream.  This
// replaces torch.mps.compile_shader + lib.<kernel>(..., threads=) of the reference (conv.py:247, 264, 269, 280;
// symmetric.py:140, 154, 165).
//
// The library links libamdhip64.so.7 / libhiprtc.so.7 by soname; loaded into a process that has imported torch, the
// dynamic linker resolves them to torch's bundled copies, so modules, streams and allocations share one HIP
// runtime.  mh_hip_runtime_path() reports which file was bound so the Python side can verify it.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/mace_hip.h"

namespace {

thread_local std::string g_err;
// launch log (mh_launch_log): bound names of the kernels launched by any thread of the process (the autograd
// engine runs backward passes on threads of its own)
std::mutex g_log_mu;
bool g_log_on = false;
std::string g_log;

struct Kernel {
    hipFunction_t fn = nullptr;
    std::string name;                      // the symbol bound to this slot
    int block = 0;
    int rows_per_block = 1;
    int grid_y = 1;          // second grid dimension (a fixed count: output blocks of a node linear)
};

}  // namespace

struct mh_module {
    hipModule_t mod = nullptr;
    int device = -1;
    Kernel k[MH_NUM_KINDS];
};

namespace {

int fail(int code, const std::string& what) {
    g_err = what;
    return code ? code : -1;
}

int hip_fail(hipError_t e, const char* what) {
    std::ostringstream os;
    os << what << ": " << hipGetErrorName(e) << " (" << hipGetErrorString(e) << ")";
    return fail(static_cast<int>(e), os.str());
}

#define MH_HIP(call)                                   \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

// Launch `kind` over `rows` rows; args are the kernel's parameters in order.
int launch(mh_module* m, int kind, int64_t rows, void** args, void* stream, const char* what) {
    if (!m) return fail(-1, std::string(what) + ": null module");
    const Kernel& k = m->k[kind];
    if (!k.fn) return fail(-1, std::string(what) + ": kernel slot not bound in this module");
    if (rows < 0) return fail(-1, std::string(what) + ": negative size");
    if (rows == 0) return 0;
    int dev = -1;
    MH_HIP(hipGetDevice(&dev));
    if (dev != m->device) {
        std::ostringstream os;
        os << what << ": module was loaded on device " << m->device << " but device " << dev << " is current";
        return fail(-1, os.str());
    }
    int64_t grid = (rows + k.rows_per_block - 1) / k.rows_per_block;
    if (grid > 0x7fffffffLL) return fail(-1, std::string(what) + ": launch too large");
    hipError_t e = hipModuleLaunchKernel(k.fn, static_cast<unsigned>(grid), static_cast<unsigned>(k.grid_y), 1,
                                         static_cast<unsigned>(k.block), 1, 1, 0, static_cast<hipStream_t>(stream), args,
                                         nullptr);
    if (e != hipSuccess) return hip_fail(e, what);
    {
        std::lock_guard<std::mutex> lock(g_log_mu);
        if (g_log_on) {
            g_log += k.name;
            g_log += ';';
        }
    }
    return 0;
}

// Launch `kind` on an explicit 1-D grid of `blocks` workgroups (kernels that size their own grid).
int launch_blocks(mh_module* m, int kind, int64_t blocks, void** args, void* stream, const char* what) {
    if (!m) return fail(-1, std::string(what) + ": null module");
    const Kernel& k = m->k[kind];
    if (!k.fn) return fail(-1, std::string(what) + ": kernel slot not bound in this module");
    if (blocks <= 0) return 0;
    if (blocks > 0x7fffffffLL) return fail(-1, std::string(what) + ": launch too large");
    int dev = -1;
    MH_HIP(hipGetDevice(&dev));
    if (dev != m->device) {
        std::ostringstream os;
        os << what << ": module was loaded on device " << m->device << " but device " << dev << " is current";
        return fail(-1, os.str());
    }
    hipError_t e = hipModuleLaunchKernel(k.fn, static_cast<unsigned>(blocks), 1, 1, static_cast<unsigned>(k.block), 1,
                                         1, 0, static_cast<hipStream_t>(stream), args, nullptr);
    if (e != hipSuccess) return hip_fail(e, what);
    {
        std::lock_guard<std::mutex> lock(g_log_mu);
        if (g_log_on) {
            g_log += k.name;
            g_log += ';';
        }
    }
    return 0;
}

// Workgroups of `kind` that fit on the whole device at once (occupancy x compute units), at least 1.
int resident_blocks(mh_module* m, int kind, int* out) {
    const Kernel& k = m->k[kind];
    int per_cu = 0, cus = 0;
    MH_HIP(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k.fn, k.block, 0));
    MH_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->device));
    *out = per_cu * cus > 0 ? per_cu * cus : 1;
    return 0;
}

}  // namespace

extern "C" {

const char* mh_last_error(void) { return g_err.c_str(); }

int mh_version(void) { return 42; }

int mh_launch_log(int enable) {
    std::lock_guard<std::mutex> lock(g_log_mu);
    const int was = g_log_on ? 1 : 0;
    g_log_on = enable != 0;
    if (!g_log_on) g_log.clear();
    return was;
}

size_t mh_launch_log_take(char* buf, size_t len) {
    std::lock_guard<std::mutex> lock(g_log_mu);
    const size_t n = g_log.size();
    if (buf && len) {
        const size_t c = n < len - 1 ? n : len - 1;
        std::memcpy(buf, g_log.data(), c);
        buf[c] = '\0';
        if (c == n) g_log.clear();
    }
    return n;
}

const char* mh_hip_runtime_path(void) {
    static std::string path;
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&hipModuleLaunchKernel), &info) && info.dli_fname) path = info.dli_fname;
    return path.c_str();
}

int mh_compile(const char* source, const char* options, void** code, size_t* code_size) {
    if (!source || !code || !code_size) return fail(-1, "mh_compile: null argument");
    *code = nullptr;
    *code_size = 0;
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, source, "mace_hip_layer.hip", 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS) return fail(static_cast<int>(r), std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
    std::vector<std::string> opts;
    if (options) {
        std::istringstream is(options);
        std::string o;
        while (is >> o) opts.push_back(o);
    }
    std::vector<const char*> optp;
    for (auto& o : opts) optp.push_back(o.c_str());
    r = hiprtcCompileProgram(prog, static_cast<int>(optp.size()), optp.data());
    size_t log_size = 0;
    hiprtcGetProgramLogSize(prog, &log_size);
    std::string log(log_size, '\0');
    if (log_size) hiprtcGetProgramLog(prog, &log[0]);
    if (r != HIPRTC_SUCCESS) {
        hiprtcDestroyProgram(&prog);
        return fail(static_cast<int>(r), std::string("hiprtcCompileProgram: ") + hiprtcGetErrorString(r) + "\n" + log);
    }
    size_t n = 0;
    r = hiprtcGetCodeSize(prog, &n);
    if (r != HIPRTC_SUCCESS || n == 0) {
        hiprtcDestroyProgram(&prog);
        return fail(static_cast<int>(r), "hiprtcGetCodeSize failed");
    }
    void* buf = std::malloc(n);
    if (!buf) {
        hiprtcDestroyProgram(&prog);
        return fail(-1, "mh_compile: out of host memory");
    }
    r = hiprtcGetCode(prog, static_cast<char*>(buf));
    hiprtcDestroyProgram(&prog);
    if (r != HIPRTC_SUCCESS) {
        std::free(buf);
        return fail(static_cast<int>(r), std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r));
    }
    *code = buf;
    *code_size = n;
    return 0;
}

void mh_free_code(void* code) { std::free(code); }

int mh_module_load(const void* code, size_t code_size, mh_module** out) {
    if (!code || !code_size || !out) return fail(-1, "mh_module_load: null argument");
    *out = nullptr;
    mh_module* m = new mh_module();
    hipError_t e = hipGetDevice(&m->device);
    if (e == hipSuccess) e = hipModuleLoadData(&m->mod, code);
    if (e != hipSuccess) {
        delete m;
        return hip_fail(e, "hipModuleLoadData");
    }
    *out = m;
    return 0;
}

int mh_module_unload(mh_module* m) {
    if (!m) return 0;
    hipError_t e = m->mod ? hipModuleUnload(m->mod) : hipSuccess;
    delete m;
    if (e != hipSuccess) return hip_fail(e, "hipModuleUnload");
    return 0;
}

int mh_module_bind_grid(mh_module* m, int kind, const char* name, int block_threads, int rows_per_block,
                        int grid_y) {
    if (!m || !name) return fail(-1, "mh_module_bind: null argument");
    if (kind < 0 || kind >= MH_NUM_KINDS) return fail(-1, "mh_module_bind: bad kernel kind");
    if (block_threads <= 0 || block_threads > 1024 || block_threads % 64 || rows_per_block <= 0 || grid_y <= 0 ||
        grid_y > 65535)
        return fail(-1, "mh_module_bind: bad launch shape");
    hipFunction_t fn = nullptr;
    MH_HIP(hipModuleGetFunction(&fn, m->mod, name));
    m->k[kind].fn = fn;
    m->k[kind].name = name;
    m->k[kind].block = block_threads;
    m->k[kind].rows_per_block = rows_per_block;
    m->k[kind].grid_y = grid_y;
    return 0;
}

int mh_module_bind(mh_module* m, int kind, const char* name, int block_threads, int rows_per_block) {
    return mh_module_bind_grid(m, kind, name, block_threads, rows_per_block, 1);
}

int mh_conv_fwd(mh_module* m, const float* x, const float* Y, const float* W, const int32_t* rowptr,
                const int32_t* eids, const int32_t* senders, float* out, int32_t N, void* stream) {
    void* args[] = {&x, &Y, &W, &rowptr, &eids, &senders, &out, &N};
    return launch(m, MH_CONV_FWD, N, args, stream, "mh_conv_fwd");
}

int mh_conv_fwd_cut_rows(mh_module* m, const float* x, const float* Y, const float* W, const int32_t* rowptr,
                         const int32_t* eids, const int32_t* senders, const float* cutoff, const int32_t* wrow,
                         float* out, int32_t N, void* stream) {
    if (!cutoff) return fail(-1, "mh_conv_fwd_cut: cutoff is NULL");
    void* args[] = {&x, &Y, &W, &rowptr, &eids, &senders, &out, &N, &cutoff, &wrow};
    // a row map: the kernel variant whose W0 loads are cacheable (shared rows are read twice)
    return launch(m, wrow ? MH_CONV_FWD_CR : MH_CONV_FWD_C, N, args, stream, "mh_conv_fwd_cut");
}

int mh_conv_fwd_cut(mh_module* m, const float* x, const float* Y, const float* W, const int32_t* rowptr,
                    const int32_t* eids, const int32_t* senders, const float* cutoff, float* out, int32_t N,
                    void* stream) {
    return mh_conv_fwd_cut_rows(m, x, Y, W, rowptr, eids, senders, cutoff, nullptr, out, N, stream);
}

int mh_conv_bwd(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                const int32_t* rowptr_s, const int32_t* eids_s, const int32_t* receivers, float* gx, float* gW,
                float* gY, int32_t N, int32_t flags, void* stream) {
    if ((flags & MH_WANT_GX) && !gx) return fail(-1, "mh_conv_bwd: gx requested but NULL");
    if ((flags & MH_WANT_GWY) && (!gW || !gY || !x)) return fail(-1, "mh_conv_bwd: gW/gY requested but NULL");
    if (!(flags & (MH_WANT_GX | MH_WANT_GWY))) return 0;
    void* args[] = {&x, &g, &Y, &W, &rowptr_s, &eids_s, &receivers, &gx, &gW, &gY, &N, &flags};
    return launch(m, MH_CONV_BWD, N, args, stream, "mh_conv_bwd");
}

int mh_conv_bwd_recv_rows(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                          const int32_t* rowptr_r, const int32_t* eids_r, const int32_t* senders,
                          const int32_t* rowptr_s, const int32_t* eids_s, float* work, float* gx, float* gW, float* gY,
                          const float* cutoff, float* g_cutoff, const int32_t* wrow, int32_t N, int32_t flags,
                          void* stream) {
    if (wrow && !cutoff) return fail(-1, "mh_conv_bwd_recv: a W0 row map needs the factored form (cutoff)");
    if (!(flags & MH_WANT_GWY)) return fail(-1, "mh_conv_bwd_recv: flags must include MH_WANT_GWY");
    if (!x || !gW || !gY) return fail(-1, "mh_conv_bwd_recv: x, gW and gY are required");
    if (cutoff && !g_cutoff) return fail(-1, "mh_conv_bwd_recv: cutoff given but g_cutoff is NULL");
    const bool masked = (flags & MH_CUT_MASKED) != 0;
    if (masked && !cutoff) return fail(-1, "mh_conv_bwd_recv: MH_CUT_MASKED needs the factored form (cutoff)");
    const bool nozero = (flags & MH_CUT_NOZERO) != 0;
    if (nozero && !masked) return fail(-1, "mh_conv_bwd_recv: MH_CUT_NOZERO needs MH_CUT_MASKED");
    const bool want_gx = (flags & MH_WANT_GX) != 0;
    if (want_gx && (!gx || !work || !rowptr_s || !eids_s))
        return fail(-1, "mh_conv_bwd_recv: gx requested but gx, work or the sender CSR is NULL");
    int32_t kflags = (want_gx ? 1 : 0) | (masked ? 2 : 0) | (nozero ? 4 : 0);
    int rc;
    if (cutoff) {
        void* args[] = {&x, &g, &Y, &W, &rowptr_r, &eids_r, &senders, &gW, &gY, &work, &N, &kflags, &cutoff,
                        &g_cutoff, &wrow};
        rc = launch(m, MH_CONV_BWD_RC, N, args, stream, "mh_conv_bwd_recv (factored weights)");
    } else {
        void* args[] = {&x, &g, &Y, &W, &rowptr_r, &eids_r, &senders, &gW, &gY, &work, &N, &kflags};
        rc = launch(m, MH_CONV_BWD_R, N, args, stream, "mh_conv_bwd_recv");
    }
    if (rc || !want_gx) return rc;
    const float* msg = work;
    const float* mask = masked ? cutoff : nullptr;      // masked edges wrote no message
    void* args2[] = {&msg, &rowptr_s, &eids_s, &gx, &N, &mask};
    return launch(m, MH_CONV_GXSUM, N, args2, stream, "mh_conv_bwd_recv (dX sum)");
}

int mh_conv_bwd_recv(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                     const int32_t* rowptr_r, const int32_t* eids_r, const int32_t* senders,
                     const int32_t* rowptr_s, const int32_t* eids_s, float* work, float* gx, float* gW, float* gY,
                     const float* cutoff, float* g_cutoff, int32_t N, int32_t flags, void* stream) {
    return mh_conv_bwd_recv_rows(m, x, g, Y, W, rowptr_r, eids_r, senders, rowptr_s, eids_s, work, gx, gW, gY,
                                 cutoff, g_cutoff, nullptr, N, flags, stream);
}

int mh_conv_bwd_x(mh_module* m, const float* g, const float* Y, const float* W, const int32_t* rowptr_s,
                  const int32_t* eids_s, const int32_t* receivers, float* gx, int32_t N, void* stream) {
    return mh_conv_bwd(m, nullptr, g, Y, W, rowptr_s, eids_s, receivers, gx, nullptr, nullptr, N, MH_WANT_GX, stream);
}

int mh_conv_bwd_wy(mh_module* m, const float* x, const float* g, const float* Y, const float* W,
                   const int32_t* senders, const int32_t* receivers, float* gW, float* gY, int32_t E, void* stream) {
    void* args[] = {&x, &g, &Y, &W, &senders, &receivers, &gW, &gY, &E};
    return launch(m, MH_CONV_BWD_WY, E, args, stream, "mh_conv_bwd_wy");
}

int mh_sc_fwd(mh_module* m, const float* X, const int32_t* elem, const float* T, float* out, int32_t N,
              void* stream) {
    void* args[] = {&X, &elem, &T, &out, &N};
    return launch(m, MH_SC_FWD, N, args, stream, "mh_sc_fwd");
}

int mh_sc_bwd(mh_module* m, const float* X, const int32_t* elem, const float* T, const float* G, float* GX,
              int32_t N, void* stream) {
    void* args[] = {&X, &elem, &T, &G, &GX, &N};
    return launch(m, MH_SC_BWD, N, args, stream, "mh_sc_bwd");
}

int mh_sc_fwd_sorted(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     float* out, int32_t N, void* stream) {
    void* args[] = {&X, &elem, &order, &T, &out, &N};
    return launch(m, MH_SC_FWD_G, N, args, stream, "mh_sc_fwd_sorted");
}

int mh_sc_bwd_sorted(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     const float* G, float* GX, int32_t N, void* stream) {
    void* args[] = {&X, &elem, &order, &T, &G, &GX, &N};
    return launch(m, MH_SC_BWD_G, N, args, stream, "mh_sc_bwd_sorted");
}

int mh_sc_fwd_irreps(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     float* out, int32_t N, void* stream) {
    if (!order) {
        void* args[] = {&X, &elem, &T, &out, &N};
        return launch(m, MH_SC_FWD_I, N, args, stream, "mh_sc_fwd_irreps");
    }
    void* args[] = {&X, &elem, &order, &T, &out, &N};
    return launch(m, MH_SC_FWD_GI, N, args, stream, "mh_sc_fwd_irreps");
}

int mh_sc_bwd_irreps(mh_module* m, const float* X, const int32_t* elem, const int32_t* order, const float* T,
                     const float* G, float* GX, int32_t N, void* stream) {
    if (!order) {
        void* args[] = {&X, &elem, &T, &G, &GX, &N};
        return launch(m, MH_SC_BWD_I, N, args, stream, "mh_sc_bwd_irreps");
    }
    void* args[] = {&X, &elem, &order, &T, &G, &GX, &N};
    return launch(m, MH_SC_BWD_GI, N, args, stream, "mh_sc_bwd_irreps");
}

int mh_sc_fwd_staged(mh_module* m, const float* X, const int32_t* slots, int32_t nslots, const int32_t* elem,
                     const float* TS, float* out, int32_t N, int32_t layout, void* stream) {
    if (layout != 0 && layout != 1) return fail(-1, "mh_sc_fwd_staged: layout must be 0 or 1");
    const int kind = layout ? MH_SC_FWD_SI : MH_SC_FWD_S;
    if (m && m->k[kind].fn && nslots % m->k[kind].rows_per_block != 0)
        return fail(-1, "mh_sc_fwd_staged: nslots must be a multiple of the workgroup's slot count");
    if (N <= 0) return 0;
    void* args[] = {&X, &slots, &elem, &TS, &out, &N};
    return launch(m, kind, nslots, args, stream, "mh_sc_fwd_staged");
}

int mh_sc_bwd_staged(mh_module* m, const float* X, const int32_t* slots, int32_t nslots, const int32_t* elem,
                     const float* TS, const float* G, float* GX, int32_t N, int32_t layout, void* stream) {
    if (layout != 0 && layout != 1) return fail(-1, "mh_sc_bwd_staged: layout must be 0 or 1");
    const int kind = layout ? MH_SC_BWD_SI : MH_SC_BWD_S;
    if (m && m->k[kind].fn && nslots % m->k[kind].rows_per_block != 0)
        return fail(-1, "mh_sc_bwd_staged: nslots must be a multiple of the workgroup's slot count");
    if (N <= 0) return 0;
    void* args[] = {&X, &slots, &elem, &TS, &G, &GX, &N};
    return launch(m, kind, nslots, args, stream, "mh_sc_bwd_staged");
}

int mh_sc_jvp(mh_module* m, const float* X, const float* V, const int32_t* elem, const float* T, float* out,
              int32_t N, int32_t layout, void* stream) {
    if (layout != 0 && layout != 1) return fail(-1, "mh_sc_jvp: layout must be 0 or 1");
    void* args[] = {&X, &V, &elem, &T, &out, &N};
    return launch(m, layout ? MH_SC_JVP_I : MH_SC_JVP, N, args, stream, "mh_sc_jvp");
}

int mh_sc_bwd2(mh_module* m, const float* X, const float* V, const int32_t* elem, const float* T, const float* G,
               float* GX, int32_t N, int32_t layout, void* stream) {
    if (layout != 0 && layout != 1) return fail(-1, "mh_sc_bwd2: layout must be 0 or 1");
    void* args[] = {&X, &V, &elem, &T, &G, &GX, &N};
    return launch(m, layout ? MH_SC_BWD2_I : MH_SC_BWD2, N, args, stream, "mh_sc_bwd2");
}

int mh_graph_build(mh_module* m, const int64_t* edge_index, int64_t E, int32_t n, int32_t* keys, int32_t* rowptr,
                   int32_t* eids, int32_t* work, int32_t* bad, void* stream) {
    if (E < 0 || n < 0 || E >= 0x7fffffffLL || n >= 0x7fffffff) return fail(-1, "mh_graph_build: bad sizes");
    if (E > 0 && n == 0) return fail(-1, "mh_graph_build: edges over zero nodes");
    if (!rowptr || !work || !bad || (E > 0 && (!edge_index || !keys || !eids)))
        return fail(-1, "mh_graph_build: NULL operand");
    int32_t* cnt = work;                         // [2, n + 1]
    int32_t* cursor = work + 2 * (int64_t)(n + 1);   // [2, n + 1]
    int32_t* tmp = work + 4 * (int64_t)(n + 1);      // [2, E]
    int rc;
    {
        void* args[] = {&cnt, &bad, &n};
        if ((rc = launch(m, MH_CSR_FILL, (int64_t)n + 1, args, stream, "mh_graph_build"))) return rc;
    }
    {
        void* args[] = {&edge_index, &keys, &cnt, &bad, &E, &n};
        if ((rc = launch(m, MH_CSR_COUNT, E, args, stream, "mh_graph_build"))) return rc;
    }
    {
        void* args[] = {&cnt, &rowptr, &cursor, &n};
        if ((rc = launch(m, MH_CSR_SCAN, 1, args, stream, "mh_graph_build"))) return rc;
    }
    {
        void* args[] = {&keys, &cursor, &tmp, &E, &n};
        if ((rc = launch(m, MH_CSR_SCATTER, E, args, stream, "mh_graph_build"))) return rc;
    }
    {
        void* args[] = {&rowptr, &tmp, &E, &n};
        if ((rc = launch(m, MH_CSR_SORT, n, args, stream, "mh_graph_build"))) return rc;
    }
    void* args[] = {&keys, &rowptr, &tmp, &eids, &E, &n};
    return launch(m, MH_CSR_RANK, E, args, stream, "mh_graph_build");
}

namespace {

// Byte offsets of the neighbour list's scratch arrays (each 256-byte aligned).
struct NLWork {
    size_t prmd, prmi, abin, bcnt, bstart, cursor, pbin, cnt, start, tot, sbase, keys, total;
};

NLWork nl_work(int64_t B, int64_t N, int64_t e_total) {
    NLWork w{};
    size_t off = 0;
    auto take = [&off](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) / 256 * 256;
        return at;
    };
    const int64_t nbins = N + B + 1;
    w.prmd = take(16 * 8 * B);
    w.prmi = take(16 * 4 * B);
    w.abin = take(4 * N);
    w.bcnt = take(4 * nbins);
    w.bstart = take(4 * nbins);
    w.cursor = take(4 * nbins);
    w.pbin = take(32 * N);
    w.cnt = take(8 * N);
    w.start = take(8 * N);
    w.tot = take(8 * B);
    w.sbase = take(8 * B);
    w.keys = take(8 * (e_total > 0 ? e_total : 0));
    w.total = off;
    return w;
}

}  // namespace

size_t mh_neighbour_list_work_size(int32_t B, int32_t N, int64_t e_total) {
    if (B < 0 || N < 0 || e_total < 0) return 0;
    return nl_work(B, N, e_total).total;
}

int mh_neighbour_list(mh_module* m, const double* pos, const double* cell, const int32_t* pbc, const int64_t* ptr,
                      int32_t B, int32_t N, double r_max, int64_t e_pad, int64_t e_total, int64_t* edge_index,
                      void* unit_shifts, void* shifts, int32_t out_f64, int32_t* n_edges, void* work, void* stream) {
    if (B < 0 || N < 0 || e_pad < 0 || e_total < 0 || static_cast<int64_t>(N) + B + 1 >= 0x7fffffffLL)
        return fail(-1, "mh_neighbour_list: bad sizes");
    if (!(r_max > 0.0) || r_max > 1e300) return fail(-1, "mh_neighbour_list: r_max must be positive and finite");
    if (e_pad > 0 && e_total != static_cast<int64_t>(B) * e_pad)
        return fail(-1, "mh_neighbour_list: with e_pad > 0, e_total must be B * e_pad");
    if (B == 0) return 0;
    if (!cell || !pbc || !ptr || !n_edges || !work || (N > 0 && !pos))
        return fail(-1, "mh_neighbour_list: NULL operand");
    if (edge_index && e_total > 0 && (!unit_shifts || !shifts))
        return fail(-1, "mh_neighbour_list: edge_index given without unit_shifts / shifts");
    const NLWork w = nl_work(B, N, e_total);
    char* base = static_cast<char*>(work);
    double* prmd = reinterpret_cast<double*>(base + w.prmd);
    int32_t* prmi = reinterpret_cast<int32_t*>(base + w.prmi);
    int32_t* abin = reinterpret_cast<int32_t*>(base + w.abin);
    int32_t* bcnt = reinterpret_cast<int32_t*>(base + w.bcnt);
    int32_t* bstart = reinterpret_cast<int32_t*>(base + w.bstart);
    int32_t* cursor = reinterpret_cast<int32_t*>(base + w.cursor);
    double* pbin = reinterpret_cast<double*>(base + w.pbin);
    int64_t* cnt = reinterpret_cast<int64_t*>(base + w.cnt);
    int64_t* start = reinterpret_cast<int64_t*>(base + w.start);
    int64_t* tot = reinterpret_cast<int64_t*>(base + w.tot);
    int64_t* sbase = reinterpret_cast<int64_t*>(base + w.sbase);
    int64_t* keys = reinterpret_cast<int64_t*>(base + w.keys);
    const int32_t nbins = N + B;
    int64_t nzero = static_cast<int64_t>(nbins) + 1;
    const char* what = "mh_neighbour_list";
    int rc;
    {
        void* args[] = {&pos, &cell, &pbc, &ptr, &B, &r_max, &prmd, &prmi};
        if ((rc = launch(m, MH_NL_SETUP, B, args, stream, what))) return rc;
    }
    {
        void* args[] = {&bcnt, &nzero};
        if ((rc = launch(m, MH_NL_ZERO, nzero, args, stream, what))) return rc;
    }
    {
        void* args[] = {&pos, &ptr, &B, &N, &prmd, &prmi, &abin, &bcnt};
        if ((rc = launch(m, MH_NL_BINS, N, args, stream, what))) return rc;
    }
    {
        int32_t nb = nbins;
        void* args[] = {&bcnt, &bstart, &cursor, &nb};
        if ((rc = launch(m, MH_NL_SCAN, 1, args, stream, what))) return rc;
    }
    {
        void* args[] = {&pos, &abin, &cursor, &pbin, &N};
        if ((rc = launch(m, MH_NL_PLACE, N, args, stream, what))) return rc;
    }
    {
        void* args[] = {&pos, &ptr, &B, &N, &prmd, &prmi, &bstart, &pbin, &r_max, &cnt};
        if ((rc = launch(m, MH_NL_COUNT, N, args, stream, what))) return rc;
    }
    {
        int64_t* ei = e_total > 0 ? edge_index : nullptr;
        void* args[] = {&ptr, &B, &N, &prmi, &cnt, &e_pad, &e_total, &start, &tot, &n_edges, &ei, &unit_shifts,
                        &shifts, &out_f64};
        if ((rc = launch(m, MH_NL_OFFSETS, B, args, stream, what))) return rc;
    }
    if (!edge_index || e_total == 0) return 0;
    {
        void* args[] = {&tot, &B, &e_pad, &sbase};
        if ((rc = launch(m, MH_NL_BASES, 1, args, stream, what))) return rc;
    }
    void* args[] = {&pos, &ptr, &B, &N, &prmd, &prmi, &bstart, &pbin, &r_max, &cnt, &start, &tot, &sbase, &e_pad,
                    &e_total, &keys, &edge_index, &unit_shifts, &shifts, &out_f64};
    return launch(m, MH_NL_FILL, N, args, stream, what);
}

int mh_species_order(mh_module* m, const float* attrs, int32_t N, int32_t ne, int32_t* elem, int32_t* order,
                     int32_t* slots, int32_t nslots, int32_t group, void* stream) {
    if (N < 0 || ne < 1 || ne > MH_SPECIES_MAX_ELEM || group < 1)
        return fail(-1, "mh_species_order: bad sizes (1 <= ne <= MH_SPECIES_MAX_ELEM, group >= 1)");
    const int64_t need = (static_cast<int64_t>(N) + group - 1) / group * group + static_cast<int64_t>(ne) * group;
    if (nslots < need) return fail(-1, "mh_species_order: nslots < ceil(N / group) group + ne group");
    if (N > 0 && (!attrs || !elem || !order)) return fail(-1, "mh_species_order: NULL operand");
    if (nslots > 0 && !slots) return fail(-1, "mh_species_order: NULL slots");
    void* args[] = {&attrs, &N, &ne, &elem, &order, &slots, &nslots, &group};
    return launch(m, MH_SPECIES_ORDER, 1, args, stream, "mh_species_order");
}

}  // extern "C"

// ------------------------------------------------------------------------------- allocation-free graph build
// Scratch of mh_graph_build_noalloc: the graph build's per-node counters and cursors and its per-edge staging
// (4 (n + 1) + 2 E int32) in device memory the library owns, so that the call allocates nothing.  Each GPU the
// library runs on holds its own copy until the process ends.  Host code never passes `scratch` itself (in host code
// the name is a stand-in, not a device address): it passes the address hipGetSymbolAddress reports for the current
// device, looked up once per device.
static __device__ __align__(256) int32_t scratch[MH_GRAPH_SCRATCH_INTS];

namespace {

std::mutex g_scratch_mu;
std::vector<int32_t*> g_scratch_ptr;       // per device ordinal: scratch's device address, null until looked up

// scratch's address on device `dev`, looked up (with `dev` made current for the lookup) on first use
int scratch_of_device(int dev, int32_t** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (dev < 0) return fail(-1, "mh_graph_build_noalloc: bad device ordinal");
    if (static_cast<int>(g_scratch_ptr.size()) <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        MH_HIP(hipGetDevice(&cur));
        if (cur != dev) MH_HIP(hipSetDevice(dev));
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) MH_HIP(hipSetDevice(cur));
        if (e != hipSuccess) return hip_fail(e, "mh_graph_build_noalloc: hipGetSymbolAddress");
        if (!p) return fail(-1, "mh_graph_build_noalloc: hipGetSymbolAddress gave a null scratch address");
        g_scratch_ptr[dev] = static_cast<int32_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" {

int mh_graph_build_noalloc(mh_module* m, const int64_t* edge_index, int64_t E, int32_t n, int32_t* keys,
                           int32_t* rowptr, int32_t* eids, int32_t* bad, void* stream) {
    if (E < 0 || n < 0 || E >= 0x7fffffffLL || n >= 0x7fffffff)
        return fail(-1, "mh_graph_build_noalloc: bad sizes");
    const int64_t need = 4 * (static_cast<int64_t>(n) + 1) + 2 * E;
    if (need > MH_GRAPH_SCRATCH_INTS) {
        std::ostringstream os;
        os << "mh_graph_build_noalloc: " << E << " edges over " << n << " nodes need " << need
           << " int32 of scratch, more than the " << MH_GRAPH_SCRATCH_INTS
           << " the library holds (use mh_graph_build with a caller-owned work buffer)";
        return fail(-1, os.str());
    }
    if (!m) return fail(-1, "mh_graph_build_noalloc: NULL module");
    // the scratch of the GPU the work is queued on: the stream's device, which must be the module's
    int dev = -1;
    MH_HIP(hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev));
    if (dev != m->device) {
        std::ostringstream os;
        os << "mh_graph_build_noalloc: the stream is on device " << dev << ", the module on device " << m->device;
        return fail(-1, os.str());
    }
    int32_t* work = nullptr;
    if (int rc = scratch_of_device(dev, &work)) return rc;
    return mh_graph_build(m, edge_index, E, n, keys, rowptr, eids, work, bad, stream);
}

int mh_sh_fwd(mh_module* m, const float* vec, float* Y, int64_t E, void* stream) {
    void* args[] = {&vec, &Y, &E};
    return launch(m, MH_SH_FWD, E, args, stream, "mh_sh_fwd");
}

int mh_sh_bwd(mh_module* m, const float* vec, const float* gY, float* gvec, int64_t E, void* stream) {
    void* args[] = {&vec, &gY, &gvec, &E};
    return launch(m, MH_SH_BWD, E, args, stream, "mh_sh_bwd");
}

int mh_sh_jvp(mh_module* m, const float* vec, const float* dvec, float* dY, int64_t E, void* stream) {
    if (E > 0 && (!vec || !dvec || !dY)) return fail(-1, "mh_sh_jvp: NULL operand");
    void* args[] = {&vec, &dvec, &dY, &E};
    return launch(m, MH_SH_JVP, E, args, stream, "mh_sh_jvp");
}

int mh_sh_bwd2(mh_module* m, const float* vec, const float* dvec, const float* gY, float* gvec, int64_t E,
               void* stream) {
    if (E > 0 && (!vec || !dvec || !gY || !gvec)) return fail(-1, "mh_sh_bwd2: NULL operand");
    void* args[] = {&vec, &dvec, &gY, &gvec, &E};
    return launch(m, MH_SH_BWD2, E, args, stream, "mh_sh_bwd2");
}

int mh_emb_jvp(mh_module* m, const float* len, const float* dlen, float* dfeats, float* dcutoff, int64_t E,
               void* stream) {
    if (E > 0 && (!len || !dlen || !dfeats || !dcutoff)) return fail(-1, "mh_emb_jvp: NULL operand");
    void* args[] = {&len, &dlen, &dfeats, &dcutoff, &E};
    return launch(m, MH_EMB_JVP, E, args, stream, "mh_emb_jvp");
}

int mh_emb_bwd2(mh_module* m, const float* len, const float* dlen, const float* gfeats, const float* gcutoff,
                float* glen, int64_t E, void* stream) {
    if (E > 0 && (!len || !dlen || !gfeats || !glen)) return fail(-1, "mh_emb_bwd2: NULL operand");
    void* args[] = {&len, &dlen, &gfeats, &gcutoff, &glen, &E};
    return launch(m, MH_EMB_BWD2, E, args, stream, "mh_emb_bwd2");
}

int mh_geom_jvp(mh_module* m, const float* vec, const float* len, const float* ggpos, const float* ggshifts,
                const int32_t* send, const int32_t* recv, const float* glen, float* dgvec, float* dglen, float* h,
                int64_t E, void* stream) {
    if (E > 0 && (!vec || !len || !send || !recv || !dgvec || !dglen || !h)) return fail(-1, "mh_geom_jvp: NULL operand");
    void* args[] = {&vec, &len, &ggpos, &ggshifts, &send, &recv, &glen, &dgvec, &dglen, &h, &E};
    return launch(m, MH_GEOM_JVP, E, args, stream, "mh_geom_jvp");
}

int mh_geom_segsum(mh_module* m, const float* g, const int32_t* perm, const int64_t* seg, float* out, int32_t B,
                   void* stream) {
    if (B < 0) return fail(-1, "mh_geom_segsum: negative structure count");
    if (B > 0 && (!g || !seg || !out)) return fail(-1, "mh_geom_segsum: NULL operand");
    void* args[] = {&g, &perm, &seg, &out, &B};
    return launch(m, MH_GEOM_SEGSUM, B, args, stream, "mh_geom_segsum");
}

int mh_geom_segsum1(mh_module* m, const float* g, const int64_t* seg, float* out, int32_t B, void* stream) {
    if (B < 0) return fail(-1, "mh_geom_segsum1: negative structure count");
    if (B > 0 && (!g || !seg || !out)) return fail(-1, "mh_geom_segsum1: NULL operand");
    void* args[] = {&g, &seg, &out, &B};
    return launch(m, MH_GEOM_SEGSUM1, B, args, stream, "mh_geom_segsum1");
}

int mh_readout_jvp(mh_module* m, const float* x, const float* v, float* de, int64_t N, void* stream) {
    if (N > 0 && (!x || !v || !de)) return fail(-1, "mh_readout_jvp: NULL operand");
    void* args[] = {&x, &v, &de, &N};
    return launch(m, MH_READOUT_JVP, N, args, stream, "mh_readout_jvp");
}

int mh_readout_bwd2(mh_module* m, const float* x, const float* v, const float* g, float* gx, int64_t N, void* stream) {
    if (N > 0 && (!x || !v || !g || !gx)) return fail(-1, "mh_readout_bwd2: NULL operand");
    void* args[] = {&x, &v, &g, &gx, &N};
    return launch(m, MH_READOUT_BWD2, N, args, stream, "mh_readout_bwd2");
}

int mh_lin_fwd_res(mh_module* m, const float* x, const float* attrs, const void* W, float* out, const int32_t* order,
                   float alpha, const float* res, int32_t N, void* stream) {
    if (N > 0 && (!x || !W || !out)) return fail(-1, "mh_lin_fwd: NULL x, W or out");
    void* args[] = {&x, &attrs, &W, &out, &N, &order, &alpha, &res};
    return launch(m, MH_LIN_FWD, N, args, stream, "mh_lin_fwd");
}

int mh_lin_fwd(mh_module* m, const float* x, const float* attrs, const void* W, float* out, const int32_t* order,
               float alpha, int32_t N, void* stream) {
    return mh_lin_fwd_res(m, x, attrs, W, out, order, alpha, nullptr, N, stream);
}

int mh_lin_bwd_sum(mh_module* m, const float* g, const float* g2, const float* g3, const float* attrs, const void* Wt,
                   float* gx, const int32_t* order, float alpha, int32_t N, void* stream) {
    if (N > 0 && (!g || !g2 || !g3 || !Wt || !gx)) return fail(-1, "mh_lin_bwd_sum: NULL g, g2, g3, Wt or gx");
    const float* res = nullptr;
    void* args[] = {&g, &attrs, &Wt, &gx, &N, &order, &alpha, &res, &g2, &g3};
    return launch(m, MH_LIN_BWD_SUM, N, args, stream, "mh_lin_bwd_sum");
}

int mh_lin_bwd(mh_module* m, const float* g, const float* attrs, const void* Wt, float* gx, const int32_t* order,
               float alpha, int32_t N, void* stream) {
    if (N > 0 && (!g || !Wt || !gx)) return fail(-1, "mh_lin_bwd: NULL g, Wt or gx");
    const float* res = nullptr;
    void* args[] = {&g, &attrs, &Wt, &gx, &N, &order, &alpha, &res};
    return launch(m, MH_LIN_BWD, N, args, stream, "mh_lin_bwd");
}

int mh_readout_fwd(mh_module* m, const float* x, float* e, int64_t N, void* stream) {
    if (N > 0 && (!x || !e)) return fail(-1, "mh_readout_fwd: NULL operand");
    void* args[] = {&x, &e, &N};
    return launch(m, MH_READOUT_FWD, N, args, stream, "mh_readout_fwd");
}

int mh_readout_bwd(mh_module* m, const float* x, const float* g, float* gx, int64_t N, void* stream) {
    if (N > 0 && (!x || !g || !gx)) return fail(-1, "mh_readout_bwd: NULL operand");
    void* args[] = {&x, &g, &gx, &N};
    return launch(m, MH_READOUT_BWD, N, args, stream, "mh_readout_bwd");
}

int mh_mlp_fwd_rows(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, float* W0, int64_t E,
                    const int32_t* rows, const int32_t* count, void* stream) {
    if (E > 0 && (!ef || !Wh || !Wl || !W0)) return fail(-1, "mh_mlp_fwd: NULL operand");
    if ((rows == nullptr) != (count == nullptr)) return fail(-1, "mh_mlp_fwd_rows: rows and count go together");
    void* args[] = {&ef, &Wh, &Wl, &W0, &E, &rows, &count};
    return launch(m, MH_MLP_FWD, E, args, stream, "mh_mlp_fwd");
}

int mh_mlp_fwd_ws(mh_module* m, const float* ef, const float* WhT, const uint16_t* Wo, float* h3, float* W0,
                  int64_t E, const int32_t* rows, const int32_t* count, int32_t ncb, void* stream) {
    if (E > 0 && (!ef || !WhT || !Wo || !h3 || !W0)) return fail(-1, "mh_mlp_fwd_ws: NULL operand");
    if ((rows == nullptr) != (count == nullptr)) return fail(-1, "mh_mlp_fwd_ws: rows and count go together");
    if (ncb < 1) return fail(-1, "mh_mlp_fwd_ws: ncb must be positive");
    if (E <= 0) return 0;
    if (!m) return fail(-1, "mh_mlp_fwd_ws: null module");
    void* a1[] = {&ef, &WhT, &h3, &E, &rows, &count};
    if (int rc = launch(m, MH_MLP_H3, E, a1, stream, "mh_mlp_fwd_ws (hidden layers)")) return rc;
    // persistent grid: 8 equal per-XCD shares of workgroups (blocks go round-robin over the XCDs), each share a
    // multiple of the ncg = ceil(ncb / 4) column groups, about as many as are resident at once
    if (!m->k[MH_MLP_OUT].fn) return fail(-1, "mh_mlp_fwd_ws: kernel slot MH_MLP_OUT not bound in this module");
    int res = 0;
    if (int rc = resident_blocks(m, MH_MLP_OUT, &res)) return rc;
    const int ncg = (ncb + 3) / 4;
    const int per_xcd = std::max(ncg, (res / 8) / ncg * ncg);
    void* a2[] = {&h3, &Wo, &W0, &E, &rows, &count};
    return launch_blocks(m, MH_MLP_OUT, 8LL * per_xcd, a2, stream, "mh_mlp_fwd_ws (output layer)");
}

int mh_mlp_fwd(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, float* W0, int64_t E, void* stream) {
    return mh_mlp_fwd_rows(m, ef, Wh, Wl, W0, E, nullptr, nullptr, stream);
}

int mh_mlp_bwd_rows(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, const float* gW0, float* gef,
                    int64_t E, const int32_t* rows, const int32_t* count, void* stream) {
    if (E > 0 && (!ef || !Wh || !Wl || !gW0 || !gef)) return fail(-1, "mh_mlp_bwd: NULL operand");
    if ((rows == nullptr) != (count == nullptr)) return fail(-1, "mh_mlp_bwd_rows: rows and count go together");
    void* args[] = {&ef, &Wh, &Wl, &gW0, &gef, &E, &rows, &count};
    return launch(m, MH_MLP_BWD, E, args, stream, "mh_mlp_bwd");
}

int mh_mlp_bwd_pairs(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, const float* gW0,
                     float* gef, int64_t E, const int32_t* rows, const int32_t* count, const int32_t* partner,
                     void* stream) {
    if (E > 0 && (!ef || !Wh || !Wl || !gW0 || !gef || !rows || !partner)) return fail(-1, "mh_mlp_bwd_pairs: NULL operand");
    if (!count) return fail(-1, "mh_mlp_bwd_pairs: NULL count");
    void* args[] = {&ef, &Wh, &Wl, &gW0, &gef, &E, &rows, &count, &partner};
    return launch(m, MH_MLP_BWD_P, E, args, stream, "mh_mlp_bwd_pairs");
}

int mh_mlp_bwd(mh_module* m, const float* ef, const float* Wh, const uint16_t* Wl, const float* gW0, float* gef,
               int64_t E, void* stream) {
    return mh_mlp_bwd_rows(m, ef, Wh, Wl, gW0, gef, E, nullptr, nullptr, stream);
}

size_t mh_edge_compact_work_size(int64_t E) {
    const int64_t nb = E > 0 ? (E + 4095) / 4096 : 1;
    return (size_t)nb * sizeof(int32_t);
}

int mh_edge_compact(mh_module* m, const float* cutoff, int64_t E, int32_t* rows, int32_t* count, void* work,
                    void* stream) {
    if (E < 0 || E >= 0x7fffffffLL) return fail(-1, "mh_edge_compact: bad edge count");
    if (!count || !work || (E > 0 && (!cutoff || !rows))) return fail(-1, "mh_edge_compact: NULL operand");
    int32_t nb = (int32_t)(E > 0 ? (E + 4095) / 4096 : 1);       // one workgroup also for E == 0: count = 0
    int32_t* bc = static_cast<int32_t*>(work);
    const int32_t* kv = nullptr;                                    // one list: the cutoff is not -0.0
    int32_t* rows2 = nullptr;
    int32_t* count2 = nullptr;
    void* a1[] = {&cutoff, &E, &bc, &kv};
    int rc = launch_blocks(m, MH_EDGE_COUNT, nb, a1, stream, "mh_edge_compact");
    if (rc) return rc;
    void* a2[] = {&cutoff, &E, &bc, &nb, &rows, &count, &kv, &rows2, &count2};
    return launch_blocks(m, MH_EDGE_PLACE, nb, a2, stream, "mh_edge_compact");
}

size_t mh_edge_pairs_work_size(int64_t E) {
    return (size_t)(E > 0 ? E : 0) * sizeof(int32_t) + 2 * mh_edge_compact_work_size(E);
}

int mh_edge_pairs(mh_module* m, const float* ef, int32_t nf, const float* cutoff, const int32_t* rowptr_r,
                  const int32_t* eids_r, const int32_t* rowptr_s, const int32_t* eids_s, const int32_t* senders,
                  const int32_t* receivers, int32_t N, int64_t E, const float* vec, int32_t* wrow, int32_t* partner,
                  int32_t* rows, int32_t* count, int32_t* srows, int32_t* scount, void* work, void* stream) {
    if (E < 0 || E >= 0x7fffffffLL || N < 0) return fail(-1, "mh_edge_pairs: bad size");
    if (nf < 1) return fail(-1, "mh_edge_pairs: nf must be at least 1");
    if (!count || !scount || !work ||
        (E > 0 && (!ef || !cutoff || !rowptr_r || !eids_r || !rowptr_s || !eids_s || !senders || !receivers ||
                   !wrow || !rows || !srows)))
        return fail(-1, "mh_edge_pairs: NULL operand");
    if ((vec == nullptr) != (partner == nullptr))
        return fail(-1, "mh_edge_pairs: vec and partner go together (both NULL or both given)");
    int32_t* keep = static_cast<int32_t*>(work);
    int32_t* bc = keep + (E > 0 ? E : 0);
    if (N > 0) {
        void* a0[] = {&ef, &nf, &cutoff, &rowptr_r, &eids_r, &rowptr_s, &eids_s, &senders, &receivers, &N, &wrow,
                      &keep, &vec, &partner};
        int rc = launch(m, MH_EDGE_PAIR, N, a0, stream, "mh_edge_pairs");
        if (rc) return rc;
    }
    // one counting pass and one placing pass build both lists: the support (srows) and the pair flags (rows)
    int32_t nb = (int32_t)(E > 0 ? (E + 4095) / 4096 : 1);
    const int32_t* kv = keep;
    void* a1[] = {&cutoff, &E, &bc, &kv};
    int rc = launch_blocks(m, MH_EDGE_COUNT, nb, a1, stream, "mh_edge_pairs");
    if (rc) return rc;
    void* a2[] = {&cutoff, &E, &bc, &nb, &srows, &scount, &kv, &rows, &count};
    return launch_blocks(m, MH_EDGE_PLACE, nb, a2, stream, "mh_edge_pairs");
}

int mh_mlp_jvp(mh_module* m, const float* ef, const float* ev, const float* Wh, const uint16_t* Wl, float* dW0,
               int64_t E, void* stream) {
    if (E > 0 && (!ef || !ev || !Wh || !Wl || !dW0)) return fail(-1, "mh_mlp_jvp: NULL operand");
    void* args[] = {&ef, &ev, &Wh, &Wl, &dW0, &E};
    return launch(m, MH_MLP_JVP, E, args, stream, "mh_mlp_jvp");
}

int mh_mlp_bwd2(mh_module* m, const float* ef, const float* ev, const float* Wh, const uint16_t* Wl, const float* gW0,
                float* gev, int64_t E, void* stream) {
    if (E > 0 && (!ef || !ev || !Wh || !Wl || !gW0 || !gev)) return fail(-1, "mh_mlp_bwd2: NULL operand");
    void* args[] = {&ef, &ev, &Wh, &Wl, &gW0, &gev, &E};
    return launch(m, MH_MLP_BWD2, E, args, stream, "mh_mlp_bwd2");
}

int mh_mlp_hid(mh_module* m, const float* ef, const float* Wh, const float* cutoff, uint16_t* hc, int64_t E,
               void* stream) {
    if (E > 0 && (!ef || !Wh || !cutoff || !hc)) return fail(-1, "mh_mlp_hid: NULL operand");
    void* args[] = {&ef, &Wh, &cutoff, &hc, &E};
    return launch(m, MH_MLP_HID, E, args, stream, "mh_mlp_hid");
}

int mh_mlp_hid_bwd(mh_module* m, const float* ef, const float* Wh, const float* gparts, int32_t nparts,
                   const float* cutoff, float* gef, float* gcut, int64_t E, void* stream) {
    if (E > 0 && (!ef || !Wh || !gparts || !cutoff || !gef || !gcut)) return fail(-1, "mh_mlp_hid_bwd: NULL operand");
    if (nparts < 1) return fail(-1, "mh_mlp_hid_bwd: nparts must be at least 1");
    void* args[] = {&ef, &Wh, &gparts, &nparts, &cutoff, &gef, &gcut, &E};
    return launch(m, MH_MLP_HIDB, E, args, stream, "mh_mlp_hid_bwd");
}

int mh_conv_fwd_mlp(mh_module* m, const float* x, const float* Y, const uint16_t* h, const float* cutoff,
                    const int32_t* rowptr, const int32_t* eids, const int32_t* senders, const uint16_t* Wf, float* out,
                    int32_t N, void* stream) {
    if (!m) return fail(-1, "mh_conv_fwd_mlp: null module");
    if (N < 0) return fail(-1, "mh_conv_fwd_mlp: negative size");
    if (N > 0 && (!x || !Y || !h || !cutoff || !rowptr || !eids || !senders || !Wf || !out))
        return fail(-1, "mh_conv_fwd_mlp: NULL operand");
    const Kernel& k = m->k[MH_CONV_FWD_M];
    const int64_t blocks = static_cast<int64_t>(k.grid_y) * ((N + k.rows_per_block - 1) / k.rows_per_block);
    void* args[] = {&x, &Y, &h, &cutoff, &rowptr, &eids, &senders, &Wf, &out, &N};
    return launch_blocks(m, MH_CONV_FWD_M, blocks, args, stream, "mh_conv_fwd_mlp");
}

int mh_conv_bwd_mlp(mh_module* m, const float* x, const float* g, const float* Y, const uint16_t* h,
                    const float* cutoff, const int32_t* eids_r, const int32_t* receivers, const int32_t* senders,
                    const int32_t* rowptr_s, const int32_t* eids_s, const uint16_t* Wf, const uint16_t* Wb,
                    float* work, float* gx, float* gY_parts, float* gh_parts, float* gY, int32_t E, int32_t N,
                    int32_t flags, void* stream) {
    if (!m) return fail(-1, "mh_conv_bwd_mlp: null module");
    if (E < 0 || N < 0) return fail(-1, "mh_conv_bwd_mlp: negative size");
    const bool want_gx = (flags & MH_WANT_GX) != 0;
    if (E > 0 && (!x || !g || !Y || !h || !cutoff || !eids_r || !receivers || !senders || !Wf || !Wb || !gY_parts ||
                  !gh_parts || !gY))
        return fail(-1, "mh_conv_bwd_mlp: NULL operand");
    if (want_gx && (!gx || (E > 0 && !work) || !rowptr_s || !eids_s))
        return fail(-1, "mh_conv_bwd_mlp: gx requested but gx, work or the sender CSR is NULL");
    const Kernel& k = m->k[MH_CONV_BWD_M];
    if (!k.fn) return fail(-1, "mh_conv_bwd_mlp: kernel slot not bound in this module");
    int rc;
    if (E > 0) {
        int resident = 1;
        if ((rc = resident_blocks(m, MH_CONV_BWD_M, &resident))) return rc;
        const int64_t tiles = (E + 15) / 16;
        const int64_t per_tile = k.grid_y;                    // channel tiles
        int64_t ngrp = resident / per_tile;
        const int64_t need = (tiles + k.rows_per_block - 1) / k.rows_per_block;
        if (ngrp > need) ngrp = need;
        if (ngrp < 1) ngrp = 1;
        int32_t ng = static_cast<int32_t>(ngrp), kflags = want_gx ? 1 : 0;
        void* args[] = {&x, &g, &Y, &h, &cutoff, &eids_r, &receivers, &senders, &Wf, &Wb, &work, &gY_parts,
                        &gh_parts, &E, &kflags, &ng};
        if ((rc = launch_blocks(m, MH_CONV_BWD_M, per_tile * ngrp, args, stream, "mh_conv_bwd_mlp"))) return rc;
        void* args2[] = {&gY_parts, &gY, &E};
        if ((rc = launch(m, MH_CONV_GYSUM, E, args2, stream, "mh_conv_bwd_mlp (gY sum)"))) return rc;
    }
    if (!want_gx) return 0;
    const float* msg = work;
    const float* mask = nullptr;
    void* args3[] = {&msg, &rowptr_s, &eids_s, &gx, &N, &mask};
    return launch(m, MH_CONV_GXSUM, N, args3, stream, "mh_conv_bwd_mlp (dX sum)");
}

int mh_emb_fwd(mh_module* m, const float* len, float* feats, float* cutoff, int64_t E, void* stream) {
    if (E > 0 && (!len || !feats || !cutoff)) return fail(-1, "mh_emb_fwd: NULL operand");
    void* args[] = {&len, &feats, &cutoff, &E};
    return launch(m, MH_EMB_FWD, E, args, stream, "mh_emb_fwd");
}

int mh_emb_bwd(mh_module* m, const float* len, const float* gfeats, const float* gcutoff, float* glen, int64_t E,
               void* stream) {
    if (E > 0 && (!len || !gfeats || !glen)) return fail(-1, "mh_emb_bwd: NULL len, gfeats or glen");
    void* args[] = {&len, &gfeats, &gcutoff, &glen, &E};
    return launch(m, MH_EMB_BWD, E, args, stream, "mh_emb_bwd");
}

int mh_edge_fwd(mh_module* m, const float* pos, const int32_t* send, const int32_t* recv, const float* shifts,
                float* vec, float* len, float* Y, float* feats, float* cutoff, int64_t E, void* stream) {
    if (E > 0 && (!pos || !send || !recv || !shifts || !vec || !len || !Y || !feats || !cutoff))
        return fail(-1, "mh_edge_fwd: NULL operand");
    void* args[] = {&pos, &send, &recv, &shifts, &vec, &len, &Y, &feats, &cutoff, &E};
    return launch(m, MH_EDGE_FWD, E, args, stream, "mh_edge_fwd");
}

int mh_edge_bwd2(mh_module* m, const float* vec, const float* len, const float* gY, const float* gfeats,
                 const float* gcutoff, const float* gY2, const float* gfeats2, const float* gcutoff2, float* gvec,
                 float* glen, int64_t E, void* stream) {
    if (E > 0 && (!vec || !len || !gY || !gfeats || !gvec || !glen)) return fail(-1, "mh_edge_bwd: NULL operand");
    void* args[] = {&vec, &len, &gY, &gfeats, &gcutoff, &gvec, &glen, &E, &gY2, &gfeats2, &gcutoff2};
    return launch(m, MH_EDGE_BWD, E, args, stream, "mh_edge_bwd");
}

int mh_edge_bwd(mh_module* m, const float* vec, const float* len, const float* gY, const float* gfeats,
                const float* gcutoff, float* gvec, float* glen, int64_t E, void* stream) {
    return mh_edge_bwd2(m, vec, len, gY, gfeats, gcutoff, nullptr, nullptr, nullptr, gvec, glen, E, stream);
}

int mh_perm_fwd(mh_module* m, const float* x, float* y, int32_t N, void* stream) {
    if (N > 0 && (!x || !y)) return fail(-1, "mh_perm_fwd: NULL operand");
    void* args[] = {&x, &y, &N};
    return launch(m, MH_PERM_FWD, N, args, stream, "mh_perm_fwd");
}

int mh_perm_bwd(mh_module* m, const float* gy, float* gx, int32_t N, void* stream) {
    if (N > 0 && (!gy || !gx)) return fail(-1, "mh_perm_bwd: NULL operand");
    void* args[] = {&gy, &gx, &N};
    return launch(m, MH_PERM_BWD, N, args, stream, "mh_perm_bwd");
}

int mh_geom_fwd(mh_module* m, const float* pos, const int32_t* send, const int32_t* recv, const float* shifts,
                float* vec, float* len, int64_t E, void* stream) {
    if (E > 0 && (!pos || !send || !recv || !shifts || !vec || !len)) return fail(-1, "mh_geom_fwd: NULL operand");
    void* args[] = {&pos, &send, &recv, &shifts, &vec, &len, &E};
    return launch(m, MH_GEOM_FWD, E, args, stream, "mh_geom_fwd");
}

int mh_geom_bwd(mh_module* m, const float* vec, const float* len, const float* gvec, const float* glen,
                const int32_t* rowptr_r, const int32_t* eids_r, const int32_t* rowptr_s, const int32_t* eids_s,
                float* gpos, float* gshifts, int32_t N, void* stream) {
    if (N > 0 && (!vec || !len || !rowptr_r || !eids_r || !rowptr_s || !eids_s || !gpos))
        return fail(-1, "mh_geom_bwd: NULL operand");
    void* args[] = {&vec, &len, &gvec, &glen, &rowptr_r, &eids_r, &rowptr_s, &eids_s, &gpos, &gshifts, &N};
    return launch(m, MH_GEOM_BWD, N, args, stream, "mh_geom_bwd");
}

}  // extern "C"
