// Host runtime of the engine: loads the embedded gfx950 code object, owns
// the kernel table, and implements the C-ABI kernel entry points
// (include/rfp4.h) over hipModuleLaunchKernel.
#include "runtime.h"

#include <elf.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

// HIP's launch with start/stop events from the dispatch itself
// (hip/hip_ext.h; that header also holds device-side templates this g++
// translation unit cannot compile, so only the declaration is repeated).
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void **kernelParams, void **extra,
                                               hipEvent_t startEvent, hipEvent_t stopEvent, uint32_t flags);

extern "C" const unsigned char rfp4_hsaco_start[];
extern "C" const unsigned char rfp4_hsaco_end[];

namespace rfp4 {

static thread_local std::string t_err;
static Runtime *g_rt = nullptr;
static std::mutex g_mu;

int set_error(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

int hip_check(hipError_t e, const char *what)
{
    if (e == hipSuccess) return RFP4_OK;
    return set_error(RFP4_E_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

Runtime *runtime() { return g_rt; }

// Names of every kernel in the embedded code object.  The blob is a clang
// offload bundle ("__CLANG_OFFLOAD_BUNDLE__", u64 entry count, then per entry
// u64 offset, u64 size, u64 triple length, triple) whose amdgcn entry is an
// ELF64 code object; each kernel `k` has a descriptor symbol `k.kd`.  Every
// offset and size is checked against the blob before it is read.
static int kernel_names(const unsigned char *blob, size_t len, std::vector<std::string> *out)
{
    static const char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
    const size_t mlen = sizeof kMagic - 1;
    auto rd64 = [&](size_t off, uint64_t *v) {
        if (off > len || len - off < 8) return false;
        std::memcpy(v, blob + off, 8);
        return true;
    };
    const unsigned char *elf = nullptr;
    size_t elf_len = 0;
    if (len >= mlen && std::memcmp(blob, kMagic, mlen) == 0) {
        uint64_t n = 0;
        size_t p = mlen;
        if (!rd64(p, &n)) return set_error(RFP4_E_HIP, "code object bundle truncated");
        p += 8;
        for (uint64_t i = 0; i < n && !elf; i++) {
            uint64_t off, size, tlen;
            if (!rd64(p, &off) || !rd64(p + 8, &size) || !rd64(p + 16, &tlen)) return set_error(RFP4_E_HIP, "bundle entry truncated");
            p += 24;
            if (tlen > len - std::min(p, len)) return set_error(RFP4_E_HIP, "bundle triple out of range");
            const std::string triple((const char *)blob + p, (size_t)tlen);
            p += tlen;
            if (triple.find("amdgcn") != std::string::npos) {
                if (off > len || size > len - off) return set_error(RFP4_E_HIP, "bundle entry out of range");
                elf = blob + off;
                elf_len = (size_t)size;
            }
        }
    } else {
        elf = blob;
        elf_len = len;
    }
    if (!elf || elf_len < sizeof(Elf64_Ehdr) || std::memcmp(elf, ELFMAG, SELFMAG) != 0)
        return set_error(RFP4_E_HIP, "no amdgcn ELF code object in the embedded blob");
    Elf64_Ehdr eh;
    std::memcpy(&eh, elf, sizeof eh);
    if (eh.e_shentsize != sizeof(Elf64_Shdr) || eh.e_shoff > elf_len ||
        (uint64_t)eh.e_shnum * sizeof(Elf64_Shdr) > elf_len - eh.e_shoff)
        return set_error(RFP4_E_HIP, "code object section table out of range");
    auto shdr = [&](uint32_t i) {
        Elf64_Shdr s;
        std::memcpy(&s, elf + eh.e_shoff + (size_t)i * sizeof(Elf64_Shdr), sizeof s);
        return s;
    };
    for (uint32_t i = 0; i < eh.e_shnum; i++) {
        const Elf64_Shdr sh = shdr(i);
        if (sh.sh_type != SHT_SYMTAB || sh.sh_entsize != sizeof(Elf64_Sym) || sh.sh_link >= eh.e_shnum) continue;
        const Elf64_Shdr st = shdr(sh.sh_link);
        if (sh.sh_offset > elf_len || sh.sh_size > elf_len - sh.sh_offset || st.sh_offset > elf_len ||
            st.sh_size > elf_len - st.sh_offset)
            return set_error(RFP4_E_HIP, "code object symbol table out of range");
        const char *strs = (const char *)elf + st.sh_offset;
        for (uint64_t j = 0; j < sh.sh_size / sizeof(Elf64_Sym); j++) {
            Elf64_Sym sym;
            std::memcpy(&sym, elf + sh.sh_offset + j * sizeof(Elf64_Sym), sizeof sym);
            if (sym.st_name >= st.sh_size) continue;
            const size_t maxn = (size_t)(st.sh_size - sym.st_name);
            const size_t nlen = strnlen(strs + sym.st_name, maxn);
            if (nlen == maxn || nlen < 4) continue; // unterminated or too short for "x.kd"
            const std::string name(strs + sym.st_name, nlen);
            if (name.compare(nlen - 3, 3, ".kd") == 0) out->push_back(name.substr(0, nlen - 3));
        }
    }
    if (out->empty()) return set_error(RFP4_E_HIP, "no kernel descriptors in the code object");
    return RFP4_OK;
}

// The kernel table is filled once by rfp4_init and read-only afterwards, so
// launches from several threads (and launches under stream capture) never
// touch the module or modify the map.
static thread_local std::vector<KernelTiming> *t_timing = nullptr;

void timing_install(std::vector<KernelTiming> *records) { t_timing = records; }

int launch(const char *name, dim3 grid, dim3 block, hipStream_t s, void *args, unsigned shmem)
{
    Runtime *rt = g_rt;
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    auto it = rt->fns.find(name);
    if (it == rt->fns.end()) return set_error(RFP4_E_HIP, "kernel %s is not in the code object", name);
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return RFP4_OK; // nothing to do
    void *params[] = {args};
    if (t_timing) {
        KernelTiming k{it->first.c_str(), nullptr, nullptr};
        int rc = hip_check(hipEventCreate(&k.start), "hipEventCreate");
        if (!rc) rc = hip_check(hipEventCreate(&k.stop), "hipEventCreate");
        if (!rc)
            rc = hip_check(hipExtModuleLaunchKernel(it->second, grid.x * block.x, grid.y * block.y, grid.z * block.z,
                                                    block.x, block.y, block.z, shmem, s, params, nullptr, k.start,
                                                    k.stop, 0),
                           name);
        if (rc) {
            if (k.start) hipEventDestroy(k.start);
            if (k.stop) hipEventDestroy(k.stop);
            return rc;
        }
        t_timing->push_back(k);
        return RFP4_OK;
    }
    return hip_check(hipModuleLaunchKernel(it->second, grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem, s,
                                           params, nullptr),
                     name);
}

int launch_coop(const char *name, dim3 grid, dim3 block, hipStream_t s, void *args, unsigned shmem)
{
    Runtime *rt = g_rt;
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    auto it = rt->fns.find(name);
    if (it == rt->fns.end()) return set_error(RFP4_E_HIP, "kernel %s is not in the code object", name);
    void *params[] = {args};
    KernelTiming k{it->first.c_str(), nullptr, nullptr};
    int rc = RFP4_OK;
    if (t_timing) {
        rc = hip_check(hipEventCreate(&k.start), "hipEventCreate");
        if (!rc) rc = hip_check(hipEventCreate(&k.stop), "hipEventCreate");
        if (!rc) rc = hip_check(hipEventRecord(k.start, s), "hipEventRecord");
    }
    if (!rc)
        rc = hip_check(hipModuleLaunchCooperativeKernel(it->second, grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem,
                                                        s, params),
                       name);
    if (t_timing) {
        if (!rc) rc = hip_check(hipEventRecord(k.stop, s), "hipEventRecord");
        if (rc) {
            if (k.start) hipEventDestroy(k.start);
            if (k.stop) hipEventDestroy(k.stop);
            return rc;
        }
        t_timing->push_back(k);
    }
    return rc;
}

int kernel_occupancy(const char *name, int block, unsigned shmem, int *per_cu)
{
    Runtime *rt = g_rt;
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    auto it = rt->fns.find(name);
    if (it == rt->fns.end()) return set_error(RFP4_E_HIP, "kernel %s is not in the code object", name);
    return hip_check(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, it->second, block, shmem), name);
}

} // namespace rfp4

using namespace rfp4;

extern "C" {

const char *rfp4_last_error(void) { return t_err.c_str(); }
int rfp4_version(void) { return 1; }

int rfp4_kernel_count(uint32_t *count)
{
    if (!count) return set_error(RFP4_E_INVALID, "null count");
    std::vector<std::string> names;
    int rc = kernel_names(rfp4_hsaco_start, (size_t)(rfp4_hsaco_end - rfp4_hsaco_start), &names);
    *count = rc ? 0u : (uint32_t)names.size();
    return rc;
}

int rfp4_kernel_name(uint32_t i, char *buf, size_t cap)
{
    if (!buf || cap == 0) return set_error(RFP4_E_INVALID, "null buffer");
    std::vector<std::string> names;
    int rc = kernel_names(rfp4_hsaco_start, (size_t)(rfp4_hsaco_end - rfp4_hsaco_start), &names);
    if (rc) return rc;
    if (i >= names.size()) return set_error(RFP4_E_INVALID, "kernel index %u >= %zu", i, names.size());
    if (names[i].size() + 1 > cap) return set_error(RFP4_E_CAPACITY, "name of kernel %u needs %zu bytes", i, names[i].size() + 1);
    std::memcpy(buf, names[i].c_str(), names[i].size() + 1);
    return RFP4_OK;
}

int rfp4_device_count(int *count)
{
    if (!count) return set_error(RFP4_E_INVALID, "null count");
    hipError_t e = hipGetDeviceCount(count);
    if (e != hipSuccess) {
        *count = 0;
        return set_error(RFP4_E_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
    }
    return RFP4_OK;
}

int rfp4_init(int device)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_rt) return g_rt->device == device ? RFP4_OK : set_error(RFP4_E_INVALID, "already initialised on device %d", g_rt->device);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return set_error(RFP4_E_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= n) return set_error(RFP4_E_INVALID, "device %d out of range (%d devices)", device, n);
    int rc = hip_check(hipSetDevice(device), "hipSetDevice");
    if (rc) return rc;
    hipDeviceProp_t prop;
    rc = hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (rc) return rc;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(RFP4_E_NO_DEVICE, "device %d is %s; this library holds gfx950 code only", device, prop.gcnArchName);
    Runtime *rt = new Runtime();
    rt->device = device;
    rt->num_cus = prop.multiProcessorCount;
    rt->max_lds = (size_t)prop.sharedMemPerBlock;
    rc = hip_check(hipModuleLoadData(&rt->module, rfp4_hsaco_start), "hipModuleLoadData");
    if (rc) {
        delete rt;
        return rc;
    }
    // every kernel handle now: the table is read-only from here on
    std::vector<std::string> names;
    rc = kernel_names(rfp4_hsaco_start, (size_t)(rfp4_hsaco_end - rfp4_hsaco_start), &names);
    for (size_t i = 0; i < names.size() && !rc; i++) {
        hipFunction_t f = nullptr;
        rc = hip_check(hipModuleGetFunction(&f, rt->module, names[i].c_str()), names[i].c_str());
        if (!rc) rt->fns.emplace(names[i], f);
    }
    if (rc) {
        hipModuleUnload(rt->module);
        delete rt;
        return rc;
    }
    // default workspace of the drop-in attn_decode
    rt->attn_part_floats = (size_t)kAttnMaxHeads * kAttnMaxSplits * (128 + 4); // [m, l, -, -, acc[hd]]
    rc = hip_check(hipMalloc((void **)&rt->attn_part, rt->attn_part_floats * sizeof(float)), "hipMalloc(attn workspace)");
    // split-K workspace of fp4_gemm
    if (!rc) rc = hip_check(hipMalloc((void **)&rt->gemm_part, kGemmWorkspaceWords * sizeof(float)), "hipMalloc(gemm workspace)");
    if (!rc)
        rc = hip_check(hipMemset(rt->gemm_part + kGemmPartFloats, 0, kGemmCounters * sizeof(uint32_t)), "hipMemset(gemm counters)");
    if (!rc) rc = hip_check(hipMalloc((void **)&rt->gemm_st, kGemmStBytes), "hipMalloc(gemm scale workspace)");
    // arrival counters of the in-kernel attention merge: zero between calls
    if (!rc) rc = hip_check(hipMalloc((void **)&rt->attn_counters, kAttnMaxHeads * sizeof(uint32_t)), "hipMalloc(attn counters)");
    if (!rc) rc = hip_check(hipMemset(rt->attn_counters, 0, kAttnMaxHeads * sizeof(uint32_t)), "hipMemset(attn counters)");
    // the allocation-free entry points' scratch on this device (current now)
    if (!rc) rc = noalloc_setup(device);
    if (!rc) rc = hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (rc) {
        hipFree(rt->attn_part);
        hipFree(rt->gemm_part);
        hipFree(rt->gemm_st);
        hipFree(rt->attn_counters);
        hipModuleUnload(rt->module);
        delete rt;
        return rc;
    }
    g_rt = rt;
    return RFP4_OK;
}

// Every HIP object the library holds, released in dependency order: the
// work of every stream, the engines (step graphs, their streams and device
// memory), the runtime's workspaces and the code object.  A host program
// calls it before it returns from main, so that no graph, stream, module or
// allocation of this library is left for the HIP runtime's exit-time
// teardown (which runs after tools such as rocprofv3 have finalized).
int rfp4_shutdown(void)
{
    std::lock_guard<std::mutex> lk(g_mu);
    Runtime *rt = g_rt;
    if (!rt) return RFP4_OK;
    int rc = hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize(shutdown)");
    engines_destroy_all();
    auto keep = [&rc](int r) {
        if (!rc) rc = r;
    };
    keep(hip_check(hipFree(rt->attn_part), "hipFree(attn workspace)"));
    keep(hip_check(hipFree(rt->gemm_part), "hipFree(gemm workspace)"));
    keep(hip_check(hipFree(rt->gemm_st), "hipFree(gemm scale workspace)"));
    keep(hip_check(hipFree(rt->attn_counters), "hipFree(attn counters)"));
    keep(hip_check(hipModuleUnload(rt->module), "hipModuleUnload"));
    g_rt = nullptr;
    delete rt;
    return rc;
}

int rfp4_device_info(int *num_cus, size_t *lds_per_block, int *clock_khz)
{
    if (!g_rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    hipDeviceProp_t prop;
    int rc = hip_check(hipGetDeviceProperties(&prop, g_rt->device), "hipGetDeviceProperties");
    if (rc) return rc;
    if (num_cus) *num_cus = prop.multiProcessorCount;
    if (lds_per_block) *lds_per_block = prop.sharedMemPerBlock;
    if (clock_khz) *clock_khz = prop.clockRate;
    return RFP4_OK;
}

int rfp4_stream_create(rfp4_stream_t *stream)
{
    if (!stream) return set_error(RFP4_E_INVALID, "null stream out");
    if (!g_rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    hipStream_t s;
    int rc = hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    if (!rc) *stream = (rfp4_stream_t)s;
    return rc;
}

int rfp4_stream_destroy(rfp4_stream_t stream) { return hip_check(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy"); }
int rfp4_stream_synchronize(rfp4_stream_t stream)
{
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int rfp4_malloc(void **dptr, size_t bytes)
{
    if (!dptr || bytes == 0) return set_error(RFP4_E_INVALID, "rfp4_malloc: null out or zero size");
    if (!g_rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    return hip_check(hipMalloc(dptr, bytes), "hipMalloc");
}

int rfp4_free(void *dptr) { return dptr ? hip_check(hipFree(dptr), "hipFree") : RFP4_OK; }

int rfp4_memset_zero(void *dptr, size_t bytes, rfp4_stream_t stream)
{
    if (!dptr) return set_error(RFP4_E_INVALID, "rfp4_memset_zero: null pointer");
    if (bytes % 4) return set_error(RFP4_E_INVALID, "rfp4_memset_zero: %zu bytes is not a multiple of 4", bytes);
    return fill_words((uint32_t *)dptr, bytes / 4, 0u, (hipStream_t)stream);
}

int rfp4_h2d(void *dst, const void *src, size_t bytes, rfp4_stream_t stream)
{
    if (!dst || !src) return set_error(RFP4_E_INVALID, "rfp4_h2d: null pointer");
    return hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync H2D");
}

int rfp4_d2h(void *dst, const void *src, size_t bytes, rfp4_stream_t stream)
{
    if (!dst || !src) return set_error(RFP4_E_INVALID, "rfp4_d2h: null pointer");
    int rc = hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync D2H");
    if (rc) return rc;
    return hip_check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int rfp4_event_create(rfp4_event_t *ev)
{
    if (!ev) return set_error(RFP4_E_INVALID, "null event out");
    hipEvent_t e;
    int rc = hip_check(hipEventCreate(&e), "hipEventCreate");
    if (!rc) *ev = (rfp4_event_t)e;
    return rc;
}
int rfp4_event_destroy(rfp4_event_t ev) { return hip_check(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy"); }
int rfp4_event_record(rfp4_event_t ev, rfp4_stream_t s)
{
    return hip_check(hipEventRecord((hipEvent_t)ev, (hipStream_t)s), "hipEventRecord");
}
int rfp4_event_synchronize(rfp4_event_t ev) { return hip_check(hipEventSynchronize((hipEvent_t)ev), "hipEventSynchronize"); }
int rfp4_event_elapsed_ms(float *ms, rfp4_event_t a, rfp4_event_t b)
{
    if (!ms) return set_error(RFP4_E_INVALID, "null ms");
    return hip_check(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime");
}

} // extern "C"

// ====================================================================== launchers
namespace rfp4 {

int fill_words(uint32_t *p, uint64_t n_words, uint32_t value, hipStream_t s)
{
    if (n_words == 0) return RFP4_OK;
    FillArgs a{p, n_words, value, 0};
    uint64_t blocks = (n_words + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    return launch("rfp4_fill", dim3((unsigned)blocks), dim3(256), s, &a);
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// LDS of the VALU GEMV: x at 36 floats per 32-value chunk (device/gemv.h).
uint32_t gemv_lds_bytes(uint32_t k) { return (k / 32u) * 36u * 4u; }

int gemv_check(uint32_t n, uint32_t k, const void *w, const void *sc, const float *x, const float *y)
{
    if (!w || !sc || !x || !y) return set_error(RFP4_E_INVALID, "gemv: null pointer");
    if (n == 0 || k == 0) return set_error(RFP4_E_SHAPE, "gemv: n=%u k=%u must be > 0", n, k);
    if (k % 32) return set_error(RFP4_E_SHAPE, "gemv: k=%u is not a multiple of the 32-element block", k);
    if (!aligned16(w) || !aligned16(x)) return set_error(RFP4_E_ALIGN, "gemv: w and x must be 16-byte aligned");
    if (g_rt && (size_t)gemv_lds_bytes(k) + 256u > g_rt->max_lds)
        return set_error(RFP4_E_CAPACITY, "gemv: k=%u activations (%u bytes) exceed the %zu-byte LDS plan", k,
                         gemv_lds_bytes(k), g_rt->max_lds);
    return RFP4_OK;
}

// Forced variant for tests (0 = automatic); thread-local like the error text.
static thread_local int t_force_r = 0, t_force_ns = -1, t_force_w = 0;

// Compiled (R, NS, W) variants; must match the table in kernels.hip.  E8M0
// scales have every variant the tests force; f32 scales the planner's own.
static bool gemv_has_ns(bool f32scale, int epi, int R, int ns, int W = 4)
{
    if (W != 4) // 8-wave workgroups: one-slice SwiGLU at R = 1, store at R = 2, residual at R = 1 of 1 or 3 slices
        return (W == 8 && ns == 1 && ((epi == RFP4_EPI_SWIGLU && R == 1) || (epi == RFP4_EPI_STORE && R == 2))) ||
               (W == 8 && !f32scale && epi == RFP4_EPI_RESIDUAL && R == 1 && (ns == 1 || ns == 3));
    const bool full = ns == 0 || ns == 1 || ns == 2 || ns == 3 || ns == 4 || ns == 7;
    const bool shrt = ns == 0 || ns == 1 || ns == 2;
    if (f32scale) {
        if (epi == RFP4_EPI_SWIGLU) return R == 1 && full;
        return R == 2 ? full : (R == 8 && shrt);
    }
    if (R == 1) return epi != RFP4_EPI_ARGMAX && full;
    if (R == 2) return full;
    if (R == 4) return epi == RFP4_EPI_SWIGLU ? (ns >= 0 && ns <= 3) : full;
    if (R == 8) return epi != RFP4_EPI_SWIGLU && shrt;
    return false;
}

// Rows per wave R and up-front K-slices NS for a GEMV launch.  NS = K/2048
// rounded up whenever compiled (all loads in flight at once), else the slice
// loop.  Measured on MI355X with x in conflict-free LDS (weights streamed
// from HBM, 8B / TinyLlama shapes): for the SwiGLU pair R = 1 at one slice
// (TinyLlama gate|up on 8 waves 4.56 us) and R = 2 from two slices up with
// E8M0 scales (8B gate|up 12.3 us vs 13.1 at R = 1 alone; in the 8B decode
// step at context 4096, 688 -> 700 tok/s), R = 2 elsewhere (8B down 9.5 us
// vs 11.1 at R = 4 and 10.6 at R = 1; q|k|v 5.0 vs 5.2-5.4; TinyLlama LM head
// 7.9-8.1 vs 8.3 at R = 4), except R = 1 for residual GEMVs of at most 2048
// rows (twice the workgroups of R = 2 where R = 2 gives one per CU; decode
// step, three engines of each interleaved: TinyLlama 2272 -> 2304 tok/s,
// Llama-3.2-1B 2774 -> 2777), R = 8 for wide matrices with short K (the LM
// heads: Llama-3.2-1B at R = 2 2683-2716 against 2774-2795 tok/s, TinyLlama's
// 32000 rows 2270-2292 at R = 2 against 2303-2307).
// With f32 scales (their compiled set): R = 1 for SwiGLU, R = 2 for every
// residual GEMV, the rest as E8M0.
GemvVariant gemv_variant(uint32_t n, uint32_t k, int epi, bool f32scale)
{
    int ns_needed = (int)((k + 2047u) / 2048u);
    int R;
    if (epi == RFP4_EPI_SWIGLU)
        R = f32scale || (ns_needed == 1 && gemv_has_ns(f32scale, epi, 1, ns_needed)) ? 1 : 2;
    else if (n >= 16384u && ns_needed <= 2) R = 8;
    else if (epi == RFP4_EPI_RESIDUAL && n <= 2048u && !f32scale) R = 1;
    else R = 2;
    // 8 waves per workgroup where compiled (one-slice SwiGLU at R = 1, store
    // at R = 2: K <= 2048; residual at R = 1 of one or three slices), else 4.
    // Measured in the TinyLlama decode step: 1811 -> 1836 tok/s (gate|up,
    // q|k|v and the LM head on 8 waves), 2307 -> 2338 (o and down on 8 waves).
    int W = 4;
    if (t_force_r) R = t_force_r;
    if (t_force_w) W = t_force_w;
    else if (gemv_has_ns(f32scale, epi, R, ns_needed, 8)) W = 8;
    int ns = gemv_has_ns(f32scale, epi, R, ns_needed, W) ? ns_needed : 0;
    if (t_force_ns >= 0) ns = t_force_ns;
    if (W != 4 && !gemv_has_ns(f32scale, epi, R, ns, W)) W = 4, ns = gemv_has_ns(f32scale, epi, R, ns_needed) ? ns_needed : 0;
    return GemvVariant{R, ns, W};
}

static thread_local int t_attn_merge = 0; // 0 automatic, 1 merge kernel, 2 in-kernel merge where it fits, 3 tagged (engines)

int attn_merge_mode() { return t_attn_merge; }

static thread_local int t_attn_head_split = 0; // query-head slices per KV head for new engines (0 = automatic)
int attn_head_split_mode() { return t_attn_head_split; }

static thread_local int t_qkva = 0; // engines created on this thread: 0 fused q|k|v GEMV + attention for one-split steps, 1 two launches, 2 fused wherever it fits
int qkva_mode() { return t_qkva; }

static thread_local int t_prefill_attn = 0; // 0 matrix-core prefill kernel, 1 one decode-kernel row per prompt row
static thread_local int t_prefill_waves = 0; // prefill attention waves per workgroup (0 = automatic)
static thread_local int t_prefill_pairing = 0; // 0 automatic, 1 one query tile per workgroup, 2 paired tiles
static thread_local int t_prefill_ksplit = 0; // prefill attention key groups per workgroup (0 automatic, 1, 2)
int prefill_attn_mode() { return t_prefill_attn; }
static thread_local int t_prefill_stop = -2; // stage after which the batched prefill stops (-2: none)
int prefill_stop() { return t_prefill_stop; }
static thread_local int t_prefill_swiglu = 0; // 0: SwiGLU + MXFP4 in the gate|up GEMM's epilogue where it applies, 1: the row kernel
int prefill_swiglu_mode() { return t_prefill_swiglu; }
static thread_local int t_prefill_rope = 0; // 0: RoPE + K/V cache rows in the q|k|v GEMM's epilogue where it applies, 1: the row kernel
int prefill_rope_mode() { return t_prefill_rope; }
static thread_local int t_prefill_attn_quant = 0; // 0: the attention rows quantized by the attention kernel, 1: by the row quantizer
int prefill_attn_quant_mode() { return t_prefill_attn_quant; }

bool attn_inmerge_mode(int mode, uint32_t splits)
{
    if (splits <= 1 || splits > kAttnInmergeMaxSplits) return false;
    return mode != 1;
}

bool attn_tagged_mode(int mode, uint32_t splits)
{
    // Automatic: above the last-arriver merge's splits.  Measured (graph step,
    // tok/s, merge kernel -> tagged): TinyLlama at context 1500 1835 -> 1886,
    // Llama-3.2-1B at 1200 2261 -> 2330, Llama-3-8B at 4096 (29 splits)
    // 672 -> 674.
    if (splits <= 1 || splits > kAttnTagMaxSplits) return false;
    return mode == 3 || (mode == 0 && splits > kAttnInmergeMaxSplits);
}

bool attn_inmerge(uint32_t max_splits)
{
    // In-kernel when the last split's merge is one round of loads (few
    // splits); above that, the second kernel's parallel merge is faster.
    if (max_splits <= 1 || max_splits > kAttnInmergeMaxSplits) return false;
    return t_attn_merge != 1;
}

int gemv_launch_v(const char *scale_name, int epi, const GemvArgs &args, hipStream_t s, const GemvVariant &v)
{
    static const char *epi_names[] = {"store", "resid", "swiglu", "argmax"};
    const bool f32scale = scale_name[0] == 'f';
    if (!gemv_has_ns(f32scale, epi, v.R, v.NS, v.W))
        return set_error(RFP4_E_INVALID, "gemv: no compiled variant R=%d NS=%d W=%d for %s/%s", v.R, v.NS, v.W,
                         scale_name, epi_names[epi]);
    if (v.NS > 0 && (uint32_t)v.NS * 2048u < args.k)
        return set_error(RFP4_E_INVALID, "gemv: NS=%d slices cannot cover k=%u", v.NS, args.k);
    char name[64];
    if (v.W == 4)
        snprintf(name, sizeof name, "rfp4_gemv_%s_%s_r%d_s%d", scale_name, epi_names[epi], v.R, v.NS);
    else
        snprintf(name, sizeof name, "rfp4_gemv_%s_%s_r%d_s%d_w%d", scale_name, epi_names[epi], v.R, v.NS, v.W);
    GemvArgs a = args;
    return launch(name, dim3(gemv_grid(args.n, v)), dim3(64u * (uint32_t)v.W), s, &a, gemv_lds_bytes(args.k));
}

int gemv_launch(const char *scale_name, int epi, const GemvArgs &args, hipStream_t s)
{
    return gemv_launch_v(scale_name, epi, args, s, gemv_variant(args.n, args.k, epi, scale_name[0] == 'f'));
}

} // namespace rfp4

extern "C" int rfp4_debug_attn_head_split(int hs)
{
    using namespace rfp4;
    if (hs != 0 && hs != 1 && hs != 2 && hs != 4 && hs != 8)
        return set_error(RFP4_E_INVALID, "head split must be 0 (automatic), 1, 2, 4 or 8");
    t_attn_head_split = hs;
    return RFP4_OK;
}

extern "C" int rfp4_debug_qkv_attn(int mode)
{
    using namespace rfp4;
    if (mode < 0 || mode > 2)
        return set_error(RFP4_E_INVALID, "q|k|v + attention mode must be 0 (fused for one split), 1 (two launches) or 2 "
                                         "(fused wherever the grid fits)");
    t_qkva = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_attn_merge(int mode)
{
    using namespace rfp4;
    if (mode < 0 || mode > 3)
        return set_error(RFP4_E_INVALID, "merge mode must be 0 (auto), 1 (merge kernel), 2 (in-kernel) or 3 (tagged)");
    t_attn_merge = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_gemv_waves(int waves)
{
    using namespace rfp4;
    if (waves != 0 && waves != 4 && waves != 8)
        return set_error(RFP4_E_INVALID, "waves per workgroup must be 0 (auto), 4 or 8");
    t_force_w = waves;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_waves(int waves)
{
    using namespace rfp4;
    if (waves != 0 && waves != 4 && waves != 8) return set_error(RFP4_E_INVALID, "prefill attention waves must be 0 (auto), 4 or 8");
    t_prefill_waves = waves;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_ksplit(int groups)
{
    using namespace rfp4;
    if (groups < 0 || groups > 2)
        return set_error(RFP4_E_INVALID, "prefill attention key groups must be 0 (auto), 1 (one) or 2 (two where compiled)");
    t_prefill_ksplit = groups;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_pairing(int mode)
{
    using namespace rfp4;
    if (mode < 0 || mode > 2) return set_error(RFP4_E_INVALID, "pairing mode must be 0 (auto), 1 (off) or 2 (on)");
    t_prefill_pairing = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_stop(int after)
{
    using namespace rfp4;
    if (after < -2) return set_error(RFP4_E_INVALID, "prefill stop must be -2 (off), -1 (after the embedding) or 10*layer + stage");
    t_prefill_stop = after;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_swiglu(int mode)
{
    using namespace rfp4;
    if (mode != 0 && mode != 1)
        return set_error(RFP4_E_INVALID, "prefill SwiGLU mode must be 0 (in the gate|up GEMM where it applies) or 1 (row kernel)");
    t_prefill_swiglu = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_rope(int mode)
{
    using namespace rfp4;
    if (mode != 0 && mode != 1)
        return set_error(RFP4_E_INVALID, "prefill RoPE mode must be 0 (in the q|k|v GEMM where it applies) or 1 (row kernel)");
    t_prefill_rope = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_attn_quant(int mode)
{
    using namespace rfp4;
    if (mode != 0 && mode != 1)
        return set_error(RFP4_E_INVALID, "prefill attention quantization mode must be 0 (in the attention kernel) or 1 (row quantizer)");
    t_prefill_attn_quant = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_prefill_attn(int mode)
{
    using namespace rfp4;
    if (mode != 0 && mode != 1) return set_error(RFP4_E_INVALID, "prefill attention mode must be 0 (matrix cores) or 1 (decode kernel per row)");
    t_prefill_attn = mode;
    return RFP4_OK;
}

extern "C" int rfp4_debug_gemv_variant(int rows_per_wave, int slices)
{
    using namespace rfp4;
    if (rows_per_wave < 0 || rows_per_wave > 8)
        return set_error(RFP4_E_INVALID, "rows_per_wave must be 0 (auto) or a compiled variant");
    t_force_r = rows_per_wave;
    t_force_ns = slices;
    return RFP4_OK;
}

namespace rfp4 {

uint32_t attn_head_split_for(uint32_t n_heads, uint32_t n_kv_heads, uint32_t splits, uint32_t num_cus)
{
    // Query-head slices per KV head: the most (a power of two dividing the
    // group) that keep the grid within two workgroups per CU.  Each slice
    // re-reads its KV head's rows (from cache after the first) but carries
    // 1/slices of the score and P.V arithmetic, and the extra workgroups hide
    // the load latency of short contexts.  Measured on MI355X (decode tok/s):
    // TinyLlama (8 heads per KV head, 1-5 splits) 1 / 2 / 4 / 8 slices:
    // 1836 / 1957 / 2080 / 2146; Llama-3-8B at context 4096 (29 splits)
    // 1 / 2 / 4: 671-679 / 680 / 657.
    const uint32_t g = n_heads / n_kv_heads;
    uint32_t hs = 1;
    while (hs * 2u <= g && g % (hs * 2u) == 0u && (uint64_t)n_kv_heads * splits * hs * 2u <= 2ull * num_cus) hs *= 2u;
    return hs;
}

int attn_launch(const AttnArgs &args, int kv_f16, hipStream_t s, uint32_t max_seq_for_grid, uint32_t rows)
{
    if (args.head_dim != 64 && args.head_dim != 128)
        return set_error(RFP4_E_SHAPE, "attn: head_dim %u unsupported (64 or 128)", args.head_dim);
    if (args.n_kv_heads == 0 || args.n_heads % args.n_kv_heads || args.n_heads / args.n_kv_heads > 8)
        return set_error(RFP4_E_SHAPE, "attn: %u query heads over %u KV heads (group of at most 8)", args.n_heads,
                         args.n_kv_heads);
    if (args.chunk == 0) return set_error(RFP4_E_INVALID, "attn: chunk must be positive");
    const uint32_t splits0 = (max_seq_for_grid + args.chunk - 1) / args.chunk;
    const uint32_t hs = args.head_split ? args.head_split
                                        : attn_head_split_for(args.n_heads, args.n_kv_heads, splits0 * rows,
                                                              g_rt ? (uint32_t)g_rt->num_cus : 256u);
    if ((args.n_heads / args.n_kv_heads) % hs)
        return set_error(RFP4_E_INVALID, "attn: head split %u does not divide the group of %u", hs,
                         args.n_heads / args.n_kv_heads);
    char name[48];
    snprintf(name, sizeof name, "rfp4_attn_hd%u_%s_g%u%s", args.head_dim, kv_f16 ? "f16" : "f32",
             attn_group_pad(args.n_heads / args.n_kv_heads / hs), args.tagged ? "_t" : "");
    if (rows == 0 || (rows > 1 && args.cosv)) return set_error(RFP4_E_INVALID, "attn: fused append is one row only");
    uint32_t splits = (max_seq_for_grid + args.chunk - 1) / args.chunk;
    if (splits > args.max_splits) return set_error(RFP4_E_INVALID, "attn: %u splits exceed the workspace's %u", splits, args.max_splits);
    if (args.counters && (rows != 1 || splits > kAttnInmergeMaxSplits))
        return set_error(RFP4_E_INVALID, "attn: the in-kernel merge takes one row and at most %u splits", kAttnInmergeMaxSplits);
    if (args.tagged && (rows != 1 || args.counters || splits > args.tag_splits || args.tag_splits > kAttnTagMaxSplits))
        return set_error(RFP4_E_INVALID, "attn: the tagged merge takes one row and at most %u splits (workspace: %u)",
                         kAttnTagMaxSplits, args.tag_splits);
    AttnArgs a = args;
    a.head_split = hs;
    int rc = launch(name, dim3(a.n_kv_heads * hs, splits, rows), dim3(256), s, &a);
    if (rc || splits <= 1 || a.counters || a.tagged) return rc;
    // the split states are merged by a second launch (stream order, no fence)
    return launch(args.head_dim == 64 ? "rfp4_attn_merge_hd64" : "rfp4_attn_merge_hd128", dim3(a.n_heads, 1, rows),
                  dim3(256), s, &a);
}

int attn_prefill_launch(const AttnPrefillArgs &a, uint32_t head_dim, hipStream_t s)
{
    if (!a.q || !a.kc || !a.vc || (!a.out && !a.q_codes)) return set_error(RFP4_E_INVALID, "attn prefill: null pointer");
    if (a.q_codes && (!a.q_scales || (a.q_scales_t && (a.n_heads * head_dim) % 256u)))
        return set_error(RFP4_E_INVALID, "attn prefill: quantized output needs scales (and n_heads * head_dim %% 256 == 0 "
                                         "for the step-blocked copy)");
    if (head_dim != 64 && head_dim != 128) return set_error(RFP4_E_SHAPE, "attn prefill: head_dim %u (64 or 128)", head_dim);
    if (a.n_kv_heads == 0 || a.n_heads % a.n_kv_heads || a.n_heads / a.n_kv_heads > 8)
        return set_error(RFP4_E_SHAPE, "attn prefill: %u query heads over %u KV heads (group of at most 8)", a.n_heads,
                         a.n_kv_heads);
    if (a.rows == 0) return RFP4_OK;
    const uint32_t g = attn_group_pad(a.n_heads / a.n_kv_heads);
    // 8 waves per workgroup (one 16-row tile each, twice the rows per staged
    // K/V block, 118 VGPRs) wherever that still gives every CU a workgroup
    // or the tile height does not change (8 query heads per KV head); else 4.
    // Measured: 8B prefill 2048 tokens 23.5 -> 22.3 ms, 512 tokens 8.52 ->
    // 8.76 ms (128 workgroups); TinyLlama 512 / 2048 tokens 3.02 -> 2.83 /
    // 7.69 -> 7.15 ms.
    uint32_t waves = 4u;
    {
        const uint32_t b8 = (uint32_t)attn_prefill_rows((int)g, 8), b4 = (uint32_t)attn_prefill_rows((int)g, 4);
        const uint64_t grid8 = (uint64_t)((a.rows + b8 - 1) / b8) * a.n_kv_heads;
        if (b8 == b4 || (g_rt && grid8 >= (uint64_t)g_rt->num_cus)) waves = 8u;
    }
    if (t_prefill_waves) waves = (uint32_t)t_prefill_waves;
    const uint32_t bq = (uint32_t)attn_prefill_rows((int)g, (int)waves); // prompt rows per workgroup
    const uint32_t ntiles = (a.rows + bq - 1) / bq;
    // Causal tiles differ in length (tile t walks t + 1 key ranges' worth of
    // blocks); pairing tile t with ntiles - 1 - t in one workgroup evens them
    // out wherever the halved grid still gives every CU a workgroup.
    bool paired = ntiles >= 2 && g_rt && (uint64_t)((ntiles + 1) / 2) * a.n_kv_heads >= (uint64_t)g_rt->num_cus;
    if (t_prefill_pairing) paired = t_prefill_pairing == 2;
    char name[48];
    // two key groups of 4 waves per workgroup (alternate key blocks, the
    // states merged at the end: the serial chain of blocks halves) where the
    // plan is 4 waves and groups of up to 4 heads.  Measured: 8B prefill 512
    // tokens 5.29-5.35 -> 5.18-5.24 ms; TinyLlama (8 heads, 8 waves) slower
    // split (2.21 -> 2.24 ms), so not compiled there.
    const bool ksplit = t_prefill_ksplit != 1 && waves == 4u && g < 8u;
    snprintf(name, sizeof name, "rfp4_attn_prefill_hd%u_g%u_w%u%s%s", head_dim, g, waves, a.q_codes ? "_q" : "",
             ksplit ? "_s2" : "");
    AttnPrefillArgs args = a;
    args.paired = paired ? 1u : 0u;
    const uint32_t gx = paired ? (ntiles + 1) / 2 : ntiles;
    return launch(name, dim3(gx, a.n_kv_heads), dim3(64u * waves * (ksplit ? 2u : 1u)), s, &args);
}

uint32_t attn_group_pad(uint32_t group) { return group <= 1u ? 1u : group <= 2u ? 2u : group <= 4u ? 4u : 8u; }

uint32_t attn_sub_chunk(uint32_t head_dim, uint32_t elem_bytes, uint32_t group)
{
    // tokens per workgroup step (256 threads / lanes per 16-byte-split row)
    // times the load steps each thread keeps in registers
    uint32_t lanes_per_row = head_dim * elem_bytes / 16u;
    return (256u / lanes_per_row) * (uint32_t)attn_steps_for((int)head_dim, (int)elem_bytes, (int)attn_group_pad(group));
}

static thread_local uint32_t t_force_attn_chunk = 0;

uint32_t attn_chunk_for(uint32_t n_kv_heads, uint32_t seq, uint32_t num_cus, uint32_t head_dim, uint32_t elem_bytes,
                        uint32_t group)
{
    if (t_force_attn_chunk) return t_force_attn_chunk;
    const uint32_t sub = attn_sub_chunk(head_dim, elem_bytes, group);
    const uint32_t step = 256u / (head_dim * elem_bytes / 16u);
    // A KV head whose whole context holds at most 128 KB of K/V takes one
    // split: no merge round trips, and the query-head slices of the launch
    // (attn_head_split_for) supply the workgroups.  Measured on MI355X,
    // TinyLlama decode (contexts up to 282, 72 KB per KV head): 64-token
    // splits 2146 tok/s, 128: 2187, 192: 2214, one split: 2263.
    if ((uint64_t)seq * 2u * head_dim * elem_bytes <= 128u * 1024u) return seq ? (seq + step - 1u) / step * step : step;
    // Else at most one (KV head, split) workgroup per CU and at least 64
    // tokens per split; the chunk is a whole number of workgroup steps and at
    // most one sub-chunk (one pass over registers) unless the context needs
    // more workgroups than CUs, in which case it is exactly one sub-chunk.
    // Llama-3-8B at context 4096 (2 MB per KV head): 144-token splits 672-690
    // tok/s, 96: 633, 192: 632, 288: 657.
    uint32_t splits = (seq + 63u) / 64u;
    uint32_t per_head = num_cus / n_kv_heads;
    if (per_head < 1u) per_head = 1u;
    if (splits > per_head) splits = per_head;
    if (splits < 1u) splits = 1u;
    uint32_t chunk = (seq + splits - 1u) / splits;
    chunk = (chunk + step - 1u) / step * step;
    return chunk < sub ? chunk : sub;
}

} // namespace rfp4

// ====================================================================== C-ABI kernels
extern "C" {

int fp4_gemv(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint32_t *w, const float *scales, const float *x,
             float *y)
{
    int rc = gemv_check(n, k, w, scales, x, y);
    if (rc) return rc;
    GemvArgs a{w, scales, x, y, nullptr, nullptr, n, k, 0, 0.0f};
    return gemv_launch("f32", RFP4_EPI_STORE, a, (hipStream_t)stream);
}

int mx4_gemv(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
             const float *x, float *y)
{
    int rc = gemv_check(n, k, codes, scales, x, y);
    if (rc) return rc;
    GemvArgs a{codes, scales, x, y, nullptr, nullptr, n, k, 0, 0.0f};
    return gemv_launch("e8m0", RFP4_EPI_STORE, a, (hipStream_t)stream);
}

int mx4_gemv_rmsnorm(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                     const float *x, const uint16_t *norm_w, float eps, float *y)
{
    int rc = gemv_check(n, k, codes, scales, x, y);
    if (rc) return rc;
    if (!norm_w) return set_error(RFP4_E_INVALID, "gemv_rmsnorm: null norm weights");
    GemvArgs a{codes, scales, x, y, nullptr, norm_w, n, k, 0, eps};
    return gemv_launch("e8m0", RFP4_EPI_STORE, a, (hipStream_t)stream);
}

int mx4_gemv_residual(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                      const float *x, float *x_res)
{
    int rc = gemv_check(n, k, codes, scales, x, x_res);
    if (rc) return rc;
    GemvArgs a{codes, scales, x, x_res, nullptr, nullptr, n, k, 0, 0.0f};
    return gemv_launch("e8m0", RFP4_EPI_RESIDUAL, a, (hipStream_t)stream);
}

int mx4_gemv_swiglu(rfp4_stream_t stream, uint32_t n, uint32_t k, uint32_t pair_off, const uint8_t *codes,
                    const uint8_t *scales, const float *x, float *out)
{
    int rc = gemv_check(n, k, codes, scales, x, out);
    if (rc) return rc;
    if (pair_off < n) return set_error(RFP4_E_SHAPE, "gemv_swiglu: pair_off %u overlaps the %u gate rows", pair_off, n);
    GemvArgs a{codes, scales, x, out, nullptr, nullptr, n, k, pair_off, 0.0f};
    return gemv_launch("e8m0", RFP4_EPI_SWIGLU, a, (hipStream_t)stream);
}

size_t mx4_gemv_argmax_workspace(uint32_t n) { return ((size_t)n + 7u) / 8u * 8u + 64u; /* >= one key per 8 rows */ }

// The per-workgroup keys of an argmax GEMV, then the step kernel's reduction
// on a scratch cursor after the keys (ids_cap = 0: no ids are written).
static int gemv_argmax_launch(hipStream_t s, const char *sname, const GemvArgs &args, void *workspace,
                              uint32_t *best_token)
{
    const GemvVariant v = gemv_variant(args.n, args.k, RFP4_EPI_ARGMAX, sname[0] == 'f');
    const uint32_t nb = gemv_grid(args.n, v);
    if ((size_t)nb * 8u + sizeof(StepState) > mx4_gemv_argmax_workspace(args.n))
        return set_error(RFP4_E_CAPACITY, "gemv_argmax: %u workgroup keys exceed the workspace of %zu bytes", nb,
                         mx4_gemv_argmax_workspace(args.n));
    int rc = gemv_launch_v(sname, RFP4_EPI_ARGMAX, args, s, v);
    if (rc) return rc;
    StepState *st = (StepState *)((char *)workspace + (size_t)nb * 8u);
    rc = fill_words((uint32_t *)st, sizeof(StepState) / 4, 0u, s);
    if (rc) return rc;
    StepArgs sa{args.best, st, nullptr, best_token, nb, 0};
    return launch("rfp4_step", dim3(1), dim3(1024), s, &sa);
}

int mx4_gemv_argmax(rfp4_stream_t stream, uint32_t n, uint32_t k, const uint8_t *codes, const uint8_t *scales,
                    const float *x, float *y, void *workspace, uint32_t *best_token)
{
    int rc = gemv_check(n, k, codes, scales, x, y);
    if (rc) return rc;
    if (!workspace || !best_token) return set_error(RFP4_E_INVALID, "gemv_argmax: null workspace or output");
    GemvArgs a{codes, scales, x, y, (unsigned long long *)workspace, nullptr, n, k, 0, 0.0f};
    return gemv_argmax_launch((hipStream_t)stream, "e8m0", a, workspace, best_token);
}

int rfp4_debug_gemv_fused(rfp4_stream_t stream, int epi, int scale_format, uint32_t n, uint32_t k, uint32_t pair_off,
                          const uint8_t *codes, const void *scales, const float *x, const uint16_t *norm_w,
                          float eps, float *y, void *workspace, uint32_t *best_token)
{
    int rc = gemv_check(n, k, codes, scales, x, y);
    if (rc) return rc;
    if (epi < RFP4_EPI_STORE || epi > RFP4_EPI_ARGMAX) return set_error(RFP4_E_INVALID, "gemv_fused: bad epilogue %d", epi);
    if (scale_format != RFP4_SCALE_E8M0 && scale_format != RFP4_SCALE_F32)
        return set_error(RFP4_E_INVALID, "gemv_fused: bad scale format %d", scale_format);
    if (epi == RFP4_EPI_ARGMAX && (!workspace || !best_token))
        return set_error(RFP4_E_INVALID, "gemv_fused: argmax needs a workspace and an output");
    if (epi == RFP4_EPI_SWIGLU && pair_off < n)
        return set_error(RFP4_E_SHAPE, "gemv_fused: pair_off %u overlaps the %u gate rows", pair_off, n);
    const char *sname = scale_format == RFP4_SCALE_F32 ? "f32" : "e8m0";
    GemvArgs a{codes, scales, x, y, (unsigned long long *)workspace, norm_w, n, k, pair_off, eps};
    if (epi == RFP4_EPI_ARGMAX) return gemv_argmax_launch((hipStream_t)stream, sname, a, workspace, best_token);
    return gemv_launch(sname, epi, a, (hipStream_t)stream);
}

int rfp4_debug_fp4_encode_check(rfp4_stream_t stream, int32_t se0, uint32_t n_se, unsigned long long *mismatches,
                                unsigned long long *tested)
{
    if (!mismatches || !tested) return set_error(RFP4_E_INVALID, "fp4_encode_check: null pointer");
    if (n_se == 0 || se0 < -127 || (int64_t)se0 + (int64_t)n_se - 1 > 125)
        return set_error(RFP4_E_INVALID, "fp4_encode_check: exponents %d .. %d outside -127 .. 125", se0,
                         (int)((int64_t)se0 + (int64_t)n_se - 1));
    Fp4CheckArgs a{mismatches, tested, se0, 0};
    return launch("rfp4_fp4_encode_check", dim3(2048, n_se), dim3(256), (hipStream_t)stream, &a);
}

int rmsnorm(rfp4_stream_t stream, uint32_t dim, float eps, const float *x, const float *weight, float *y)
{
    if (!x || !weight || !y) return set_error(RFP4_E_INVALID, "rmsnorm: null pointer");
    if (dim == 0) return set_error(RFP4_E_SHAPE, "rmsnorm: dim must be > 0");
    RmsnormArgs a{x, weight, y, dim, eps};
    return launch("rfp4_rmsnorm_f32w", dim3(1), dim3(1024), (hipStream_t)stream, &a);
}

int rmsnorm_f16w(rfp4_stream_t stream, uint32_t dim, float eps, const float *x, const uint16_t *weight, float *y)
{
    if (!x || !weight || !y) return set_error(RFP4_E_INVALID, "rmsnorm: null pointer");
    if (dim == 0) return set_error(RFP4_E_SHAPE, "rmsnorm: dim must be > 0");
    RmsnormArgs a{x, weight, y, dim, eps};
    return launch("rfp4_rmsnorm_f16w", dim3(1), dim3(1024), (hipStream_t)stream, &a);
}

int rope(rfp4_stream_t stream, uint32_t num_heads, uint32_t head_dim, uint32_t cos_base, const float *cos_tab,
         const float *sin_tab, float *q)
{
    if (!cos_tab || !sin_tab || !q) return set_error(RFP4_E_INVALID, "rope: null pointer");
    if (head_dim == 0 || head_dim % 2) return set_error(RFP4_E_SHAPE, "rope: head_dim %u must be even", head_dim);
    RopeArgs a{q, cos_tab, sin_tab, num_heads, head_dim, cos_base, 0};
    uint32_t total = num_heads * (head_dim / 2);
    return launch("rfp4_rope", dim3((total + 255) / 256), dim3(256), (hipStream_t)stream, &a);
}

int copy_into(rfp4_stream_t stream, uint32_t n, uint32_t off, const float *src, float *dst)
{
    if (!src || !dst) return set_error(RFP4_E_INVALID, "copy_into: null pointer");
    CopyArgs a{src, dst, n, off};
    return launch("rfp4_copy_into_f32", dim3((n + 255) / 256), dim3(256), (hipStream_t)stream, &a);
}

int kv_append_f16(rfp4_stream_t stream, uint32_t n, uint32_t off, const float *src, uint16_t *dst)
{
    if (!src || !dst) return set_error(RFP4_E_INVALID, "kv_append_f16: null pointer");
    CopyArgs a{src, dst, n, off};
    return launch("rfp4_copy_into_f16", dim3((n + 255) / 256), dim3(256), (hipStream_t)stream, &a);
}

} // extern "C"

namespace rfp4 {

int attn_decode_ws(hipStream_t s, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t seq, const float *q, const void *kc,
                   const void *vc, uint64_t ts, uint64_t hs, float *out, int f16, float *part, size_t part_floats,
                   bool allow_inmerge)
{
    Runtime *rt = runtime();
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    if (!q || !kc || !vc || !out) return set_error(RFP4_E_INVALID, "attn_decode: null pointer");
    if (nkv == 0 || nh == 0 || nh % nkv) return set_error(RFP4_E_SHAPE, "attn_decode: n_heads %u not a multiple of n_kv_heads %u", nh, nkv);
    if (nh / nkv > 8) return set_error(RFP4_E_SHAPE, "attn_decode: GQA group %u > 8", nh / nkv);
    if (seq == 0) return set_error(RFP4_E_SHAPE, "attn_decode: seq must be >= 1");
    if (nh > kAttnMaxHeads) return set_error(RFP4_E_CAPACITY, "attn_decode: %u heads > %u", nh, kAttnMaxHeads);
    uint32_t eb = f16 ? 2u : 4u;
    if (((uintptr_t)kc | (uintptr_t)vc) & 15u || (ts * eb) % 16u || (hs * eb) % 16u)
        return set_error(RFP4_E_ALIGN, "attn_decode: K/V rows must start 16-byte aligned (strides %llu, %llu)",
                         (unsigned long long)ts, (unsigned long long)hs);
    uint32_t chunk = attn_chunk_for(nkv, seq, rt->num_cus, hd, eb, nh / nkv);
    uint32_t splits = (seq + chunk - 1) / chunk;
    if (splits > kAttnMaxSplits)
        return set_error(RFP4_E_CAPACITY, "attn_decode: seq %u needs %u splits of %u tokens (> %u)", seq, splits, chunk,
                         kAttnMaxSplits);
    if (splits > 1 && (size_t)nh * splits * (hd + 4) > part_floats)
        return set_error(RFP4_E_CAPACITY, "attn_decode: %u heads x %u splits x %u floats of split state exceed the "
                                          "%zu-float workspace", nh, splits, hd + 4, part_floats);
    AttnArgs a{};
    a.q = q; a.kc = kc; a.vc = vc; a.out = out;
    a.part = part; a.pos_ptr = nullptr;
    a.ts = ts; a.hs = hs;
    a.n_heads = nh; a.n_kv_heads = nkv; a.head_dim = hd; a.seq = seq;
    a.chunk = chunk; a.max_splits = splits;
    if (allow_inmerge && attn_inmerge(splits)) a.counters = rt->attn_counters;
    return attn_launch(a, f16, s, seq, 1);
}

} // namespace rfp4

extern "C" {

// The drop-in attention calls share the library's split-state workspace and
// merge counters: calls that overlap on one device (several streams or
// threads) race on them.
static int attn_common(hipStream_t s, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t seq, const float *q,
                       const void *kc, const void *vc, uint64_t ts, uint64_t hs, float *out, int f16)
{
    Runtime *rt = runtime();
    return attn_decode_ws(s, nh, nkv, hd, seq, q, kc, vc, ts, hs, out, f16, rt ? rt->attn_part : nullptr,
                          rt ? rt->attn_part_floats : 0, true);
}

int attn_decode(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t seq, const float *q,
                const float *kc, const float *vc, float *out)
{
    return attn_common((hipStream_t)stream, n_heads, n_kv_heads, 64, seq, q, kc, vc, (uint64_t)n_kv_heads * 64u, 64u,
                       out, 0);
}

int attn_decode_f16(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq,
                    const float *q, const uint16_t *kc, const uint16_t *vc, uint64_t token_stride,
                    uint64_t head_stride, float *out)
{
    return attn_common((hipStream_t)stream, n_heads, n_kv_heads, head_dim, seq, q, kc, vc, token_stride, head_stride,
                       out, 1);
}

int attn_prefill_f16(rfp4_stream_t stream, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t pos0,
                     uint32_t rows, const float *q, uint32_t q_row_stride, const uint16_t *kc, const uint16_t *vc,
                     uint64_t token_stride, uint64_t head_stride, float *out, uint32_t out_row_stride)
{
    if (!runtime()) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    if (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15u || q_row_stride % 4u || (token_stride * 2u) % 16u)
        return set_error(RFP4_E_ALIGN, "attn_prefill_f16: q rows and K/V rows must start 16-byte aligned");
    if ((uintptr_t)out & 15u || out_row_stride % 4u)
        return set_error(RFP4_E_ALIGN, "attn_prefill_f16: out rows must start 16-byte aligned");
    if (rows && q_row_stride < n_heads * head_dim)
        return set_error(RFP4_E_SHAPE, "attn_prefill_f16: q row stride %u < %u", q_row_stride, n_heads * head_dim);
    if (rows && out_row_stride < n_heads * head_dim)
        return set_error(RFP4_E_SHAPE, "attn_prefill_f16: out row stride %u < %u", out_row_stride, n_heads * head_dim);
    AttnPrefillArgs a{q, kc, vc, out, token_stride, head_stride, q_row_stride, out_row_stride, n_heads, n_kv_heads, pos0, rows, 0u};
    return attn_prefill_launch(a, head_dim, (hipStream_t)stream);
}

int swiglu(rfp4_stream_t stream, uint32_t n, const float *gate, const float *up, float *out)
{
    if (!gate || !up || !out) return set_error(RFP4_E_INVALID, "swiglu: null pointer");
    EltwiseArgs a{gate, up, out, n, 0};
    return launch("rfp4_swiglu", dim3((n + 255) / 256), dim3(256), (hipStream_t)stream, &a);
}

int residual(rfp4_stream_t stream, uint32_t n, const float *y, float *x)
{
    if (!y || !x) return set_error(RFP4_E_INVALID, "residual: null pointer");
    EltwiseArgs a{y, nullptr, x, n, 0};
    return launch("rfp4_residual", dim3((n + 255) / 256), dim3(256), (hipStream_t)stream, &a);
}

int argmax(rfp4_stream_t stream, uint32_t n, const float *logits, uint32_t *out)
{
    if (!logits || !out) return set_error(RFP4_E_INVALID, "argmax: null pointer");
    ArgmaxArgs a{logits, out, n, 0};
    return launch("rfp4_argmax", dim3(1), dim3(1024), (hipStream_t)stream, &a);
}

int fp4_mma_allones(rfp4_stream_t stream, float *out)
{
    if (!out) return set_error(RFP4_E_INVALID, "fp4_mma_allones: null pointer");
    MmaTileArgs a{nullptr, nullptr, nullptr, nullptr, out, 0, 0};
    return launch("rfp4_mma_allones", dim3(1), dim3(64), (hipStream_t)stream, &a);
}

int fp4_quantize_absmax(const float *w, uint32_t rows, uint32_t k, uint32_t *packed, float *scales)
{
    // The reference's host packer (llama_run/src/main.rs:334-376): per block of
    // 32, scale = absmax / 6 (1 for an all-zero block), each value / scale to
    // the nearest E2M1 magnitude with ties to the smaller one, sign bit for
    // negative values, 8 codes per word, low nibble first.  Nearest-with-ties-
    // down is decided here against the midpoints of the magnitude table,
    // which the reference's scan of |a - level| reproduces exactly: near a
    // midpoint both differences are exact (Sterbenz), elsewhere they are far
    // apart.
    if (!w || !packed || !scales) return set_error(RFP4_E_INVALID, "fp4_quantize_absmax: null pointer");
    if (rows == 0 || k == 0 || k % 32) return set_error(RFP4_E_SHAPE, "fp4_quantize_absmax: k=%u must be a positive multiple of 32", k);
    static const float kMid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
    const uint32_t nb = k / 32;
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t b = 0; b < nb; b++) {
            const float *x = w + (size_t)r * k + (size_t)b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
            const float scale = amax > 0.0f ? amax / 6.0f : 1.0f;
            scales[(size_t)r * nb + b] = scale;
            uint32_t *dst = packed + ((size_t)r * k + (size_t)b * 32) / 8;
            for (int wd = 0; wd < 4; wd++) {
                uint32_t word = 0;
                for (int j = 0; j < 8; j++) {
                    const float v = x[wd * 8 + j] / scale, a = std::fabs(v);
                    uint32_t code = 0;
                    while (code < 7 && a > kMid[code]) code++;
                    if (v < 0.0f) code |= 8u;
                    word |= code << (4 * j);
                }
                dst[wd] = word;
            }
        }
    return RFP4_OK;
}

int mx4_quantize(rfp4_stream_t stream, uint64_t rows, uint64_t k, const void *src, int src_is_bf16, uint8_t *codes,
                 uint8_t *scales)
{
    return mx4_quantize_st((hipStream_t)stream, rows, k, src, src_is_bf16, codes, scales, nullptr);
}

int mx4_quantize_tiled(rfp4_stream_t stream, uint64_t rows, uint64_t k, const void *src, int src_is_bf16,
                       uint8_t *codes, uint8_t *scales, uint8_t *scales_tiled)
{
    if (!scales_tiled) return set_error(RFP4_E_INVALID, "mx4_quantize_tiled: null pointer");
    return mx4_quantize_st((hipStream_t)stream, rows, k, src, src_is_bf16, codes, scales, scales_tiled);
}

size_t mx4_scales_tiled_bytes(uint32_t rows, uint32_t k) { return scales_tiled_bytes(rows, k); }

int mx4_scales_tile(rfp4_stream_t stream, uint32_t rows, uint32_t k, const uint8_t *scales, uint8_t *scales_tiled)
{
    if (!scales || !scales_tiled) return set_error(RFP4_E_INVALID, "mx4_scales_tile: null pointer");
    if (rows == 0 || k == 0 || k % 256u) return set_error(RFP4_E_SHAPE, "mx4_scales_tile: rows=%u k=%u (k a multiple of 256)", rows, k);
    if (((uintptr_t)scales | (uintptr_t)scales_tiled) & 3u) return set_error(RFP4_E_ALIGN, "mx4_scales_tile: 4-byte alignment");
    return scales_tile_launch((hipStream_t)stream, k, scales, scales_tiled, rows, nullptr, nullptr, 0u);
}

} // extern "C"

namespace rfp4 {

int mx4_quantize_st(hipStream_t stream, uint64_t rows, uint64_t k, const void *src, int src_is_bf16, uint8_t *codes,
                    uint8_t *scales, uint8_t *scales_t)
{
    if (!src || !codes || !scales) return set_error(RFP4_E_INVALID, "mx4_quantize: null pointer");
    if (k == 0 || k % 32) return set_error(RFP4_E_SHAPE, "mx4_quantize: k=%llu not a multiple of 32", (unsigned long long)k);
    if (scales_t && (k % 256u || rows > 0xFFFFFFFFull))
        return set_error(RFP4_E_SHAPE, "mx4_quantize: the step-blocked scales need k a multiple of 256 (k=%llu)",
                         (unsigned long long)k);
    if (((uintptr_t)codes & 15u) != 0) return set_error(RFP4_E_ALIGN, "mx4_quantize: codes must be 16-byte aligned");
    if (((uintptr_t)src & (src_is_bf16 ? 7u : 15u)) != 0)
        return set_error(RFP4_E_ALIGN, "mx4_quantize: src must be %u-byte aligned", src_is_bf16 ? 8u : 16u);
    QuantMxArgs a{src, codes, scales, rows, k, scales_t};
    uint64_t blocks = (rows * (k / 4) + 255) / 256; // one thread per 4 values
    if (blocks > 65536) blocks = 65536;
    return launch(src_is_bf16 ? "rfp4_quant_mx_bf16" : "rfp4_quant_mx_f32", dim3((unsigned)blocks), dim3(256), stream, &a);
}

int scales_tile_launch(hipStream_t s, uint32_t k, const uint8_t *src0, uint8_t *dst0, uint32_t rows0,
                       const uint8_t *src1, uint8_t *dst1, uint32_t rows1)
{
    ScaleTileArgs a{{src0, src1}, {dst0, dst1}, {rows0, rows1}, k};
    const uint64_t words = (scales_tiled_bytes(rows0, k) + scales_tiled_bytes(rows1, k)) / 4u;
    const uint64_t blocks = std::min<uint64_t>((words + 255u) / 256u, 8192u);
    return launch("rfp4_scales_tile", dim3((unsigned)std::max<uint64_t>(blocks, 1u)), dim3(256), s, &a);
}

} // namespace rfp4

namespace {

struct GemmTile {
    uint32_t bm, bn;
    const char *name;
    uint32_t occ; // workgroups per CU (registers / LDS of the compiled kernel)
};
// Compiled tile shapes (kernels.hip GEMM_KERNEL), largest first.
// (occ: workgroups per CU of the double-buffered kernel as this build compiles
// it, used when no runtime is initialised; gemm_occ asks the runtime)
constexpr GemmTile kGemmTiles[] = {
    {256, 256, "rfp4_gemm_256x256", 1}, {256, 128, "rfp4_gemm_256x128", 1}, {128, 128, "rfp4_gemm_128x128", 1},
    {64, 128, "rfp4_gemm_64x128", 2},   {32, 128, "rfp4_gemm_32x128", 3},
};
constexpr int kGemmNumTiles = (int)(sizeof(kGemmTiles) / sizeof(kGemmTiles[0]));
// Workgroups of tile i's double-buffered kernel that fit one CU (registers
// and LDS of the compiled code object), asked once per process.
uint32_t gemm_occ(int i)
{
    static std::atomic<uint32_t> occ[kGemmNumTiles];
    uint32_t v = occ[i].load(std::memory_order_relaxed);
    if (v) return v;
    int per_cu = 0;
    if (!g_rt || kernel_occupancy(kGemmTiles[i].name, 256, 0, &per_cu) || per_cu <= 0) return kGemmTiles[i].occ;
    occ[i].store((uint32_t)per_cu, std::memory_order_relaxed);
    return (uint32_t)per_cu;
}
// plan index of the few-row kernel (gemm_rows.h): 16 * MA activation rows,
// 16 W rows per workgroup, at most SEG (nb) K segments of 512 per wave
constexpr int kGemmSkinny = kGemmNumTiles;
thread_local int t_gemm_tile = -1, t_gemm_kz = 0;
thread_local int t_gemm_reduce_kernel = 0; // 1: split-K sums always in the reduce kernel
thread_local int t_gemm_stages = 0; // DMA stages of the tiled GEMM (0 / 2: double buffer; 3, 4 where compiled)
thread_local int t_gemm_pp = 0;     // 0: automatic, 1: 4-wave kernels only, 2: ping-pong wherever compiled

struct GemmPlan {
    int tile;
    uint32_t kz;
    int ma = 0, nb = 0; // few-row plan only: activation fragments, K segments per wave
    int nst = 2;        // tiled plans: DMA stages of the K pipeline (kernels.hip GEMM_KERNEL_P above 2)
};


// The K pipeline for a grid of one round of one workgroup per CU: 4 stages
// for 32x128 and 64x128, 3 for 128x128; 256x128, whose pipelined K loop
// already reads the next step under this step's MFMAs, keeps double
// buffering (14336x4096 at M = 512: 25.4 vs 29.2 us with 3 stages); 256x256
// has one.  (128x128 alone measured about 6 % faster double-buffered, but
// 3 stages inside the 8B layer sequence of the config-5 stack: 3518-3530 vs
// 3593-3614 us, same process.)
int gemm_deep_stages(int tile) { return tile == 3 || tile == 4 ? 4 : tile == 2 ? 3 : 2; }

// The few-row kernel: at most 64 activation rows, K a multiple of 512 in at
// most 8 waves of up to 4 segments (2 for 64 rows).
bool gemm_skinny_ok(uint32_t m, uint32_t k)
{
    return m <= 64u && k % 512u == 0u && k / 512u <= (m <= 32u ? 32u : 16u);
}
// Measured on MI355X at m = 32 (us, HIP events; few-row kernel with 1 / 2 / 4
// W fragments per workgroup, then the tiled 32x128): 4096x4096 5.81 / 6.62 /
// 9.11, 10.11; 6144x4096 7.87 / 6.93 / 9.20, 11.60; 28672x4096 23.91 / 20.25
// / 17.70, 21.49; 4096x14336 11.66 (one fragment), 15.35; 128256x4096 91.74
// / 69.10 / 62.66, 68.67.  At m = 16 the 128256x4096 LM head 56.90 (4
// fragments) against 64.78 tiled.  The few-row kernel wins at every shape up
// to 32 rows.
bool gemm_skinny_pays(uint32_t m, uint32_t n, uint32_t k)
{
    (void)n;
    return gemm_skinny_ok(m, k) && m <= 32u;
}
// K segments per wave: the K segments over at most 8 waves
uint32_t gemm_rows_seg(uint32_t k) { return k / 512u <= 8u ? 1u : (k / 512u <= 16u ? 2u : 4u); }
// the compiled few-row variants (kernels.hip GEMM_ROWS_KERNEL): fragments
// of 16 activation rows, K segments per wave, fragments of 16 W rows
bool gemm_rows_has(int mb, int seg, int nf)
{
    if (mb <= 2) return (seg == 1 && (nf == 1 || nf == 2 || nf == 4)) || (seg == 2 && (nf == 1 || nf == 2)) || (seg == 4 && nf == 1);
    return (seg <= 2 && nf == 1) || (seg == 1 && nf == 2);
}
// W fragments per workgroup: the most (4, 2, 1) that still give three CUs in
// four a workgroup (each workgroup shares its activation loads over its W
// rows; measured above)
int gemm_rows_nf(int mb, int seg, uint32_t n, uint32_t num_cus)
{
    for (int nf = 4; nf > 1; nf /= 2)
        if (gemm_rows_has(mb, seg, nf) && 4ull * ((n + 16u * nf - 1u) / (16u * nf)) >= 3ull * num_cus) return nf;
    return 1;
}

uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Tile: the largest one that does not waste more than a quarter of its rows
// on m and still yields a tile per CU; else the smallest such tile, with the
// K split raised until every CU has a workgroup (bounded by the workspace).
// Two measured exceptions below: 256x256 at 7/8 fill, and long K split in two.
static GemmPlan gemm_plan_tile(uint32_t m, uint32_t n, uint32_t k, uint32_t num_cus)
{
    const uint32_t nsuper = k / 256u;
    if (t_gemm_tile == kGemmSkinny || (t_gemm_tile < 0 && gemm_skinny_pays(m, n, k))) {
        // few activation rows: stream W like a GEMV, 16 NF W rows per
        // workgroup (kz: NF, a forced plan may set it)
        GemmPlan p{kGemmSkinny, 1u};
        p.ma = m <= 16u ? 1 : (m <= 32u ? 2 : 4);
        p.nb = (int)gemm_rows_seg(k);
        p.kz = t_gemm_tile == kGemmSkinny && t_gemm_kz > 0 ? (uint32_t)t_gemm_kz
                                                            : (uint32_t)gemm_rows_nf(p.ma, p.nb, n, num_cus);
        return p;
    }
    int pick = t_gemm_tile;
    if (pick < 0 && m >= 1024u) {
        // many rows: the fewest rounds of resident workgroups (tiles over
        // occupancy x CUs), then the fullest last round, then the most
        // workgroups per CU.  Measured at M = 2048 (8B prefill): q|k|v 256x256
        // 49.6 us (vs 60.0 for 256x128), o and down 128x128 29.6 / 82.2 us (vs
        // 33.2 / 90.2), gate|up 256x256.
        int best = -1;
        uint64_t best_rounds = 0;
        double best_fill = 0.0;
        for (int i = 0; i < kGemmNumTiles; i++) {
            const GemmTile &t = kGemmTiles[i];
            if ((uint64_t)ceil_div(m, t.bm) * t.bm * 4u > (uint64_t)m * 5u) continue; // > 25% padding
            const uint64_t nt = (uint64_t)ceil_div(m, t.bm) * ceil_div(n, t.bn), slots = (uint64_t)gemm_occ(i) * num_cus;
            const uint64_t rounds = (nt + slots - 1) / slots;
            const double fill = (double)nt / (double)(rounds * slots);
            const bool better = best < 0 || rounds < best_rounds ||
                                (rounds == best_rounds && (fill > best_fill + 0.01 ||
                                                           (fill > best_fill - 0.01 && gemm_occ(i) > gemm_occ(best))));
            if (better) best = i, best_rounds = rounds, best_fill = fill;
        }
        // (a grid under half the CUs goes to the K-split rule below)
        if (best >= 0 && 2ull * ceil_div(m, kGemmTiles[best].bm) * ceil_div(n, kGemmTiles[best].bn) >= num_cus)
            return {best, 1u};
    }
    if (pick < 0) {
        // one round of 256x256 tiles over at least 7/8 of the CUs beats two
        // rounds of 256x128 (one workgroup per CU either way): 8B gate|up at
        // M = 512 (224 tiles) 50 vs 66 us
        const GemmTile &t = kGemmTiles[0];
        const uint64_t nt = (uint64_t)ceil_div(m, t.bm) * ceil_div(n, t.bn);
        if ((uint64_t)ceil_div(m, t.bm) * t.bm * 4u <= (uint64_t)m * 5u && nt * 8u >= 7ull * num_cus && nt < num_cus)
            return {0, 1u};
        // likewise one round of 256x128 tiles over two rounds of 128x128:
        // 14336x4096 at M = 512 25.4 us (double-buffered, pipelined loop)
        // against 32.8; 28672x4096 at M = 256 26.4 against 34.0
        const GemmTile &t1 = kGemmTiles[1];
        const uint64_t nt1 = (uint64_t)ceil_div(m, t1.bm) * ceil_div(n, t1.bn);
        if ((uint64_t)ceil_div(m, t1.bm) * t1.bm * 4u <= (uint64_t)m * 5u && nt1 * 8u >= 7ull * num_cus && nt1 < num_cus)
            return {1, 1u};
        // and one round of 128x128 tiles over at least 3/4 of the CUs over
        // 64x128 tiles past one per CU: alone about equal (6144x4096 at M =
        // 512 15.9-16.2 vs 14.9-15.2 us), but inside the 8B layer sequence
        // of the config-5 stack the q|k|v shape on 128x128 saves about 2 us
        // per layer (stack 3587 vs 3656-3670 us, same process)
        const GemmTile &t2 = kGemmTiles[2];
        const uint64_t nt2 = (uint64_t)ceil_div(m, t2.bm) * ceil_div(n, t2.bn);
        if ((uint64_t)ceil_div(m, t2.bm) * t2.bm * 4u <= (uint64_t)m * 5u && nt2 * 4u >= 3ull * num_cus && nt2 < num_cus)
            return {2, 1u};
    }
    for (int i = 0; pick < 0 && i < kGemmNumTiles; i++) {
        const GemmTile &t = kGemmTiles[i];
        if (t.bm > 32u && (uint64_t)ceil_div(m, t.bm) * t.bm * 4u > (uint64_t)m * 5u) continue; // > 25% padding
        if ((uint64_t)ceil_div(m, t.bm) * ceil_div(n, t.bn) >= num_cus || i == kGemmNumTiles - 1) pick = i;
    }
    const uint64_t tiles = (uint64_t)ceil_div(m, kGemmTiles[pick].bm) * ceil_div(n, kGemmTiles[pick].bn);
    if (t_gemm_kz > 0) return {pick, std::min<uint32_t>((uint32_t)t_gemm_kz, nsuper)};
    if (tiles >= num_cus) {
        // long K at about one workgroup per CU: two K splits let two
        // workgroups per CU overlap their serial chains of K steps (8B down
        // at M = 512: 64x128, 56 steps, 51 -> 37 us before the pipelined
        // loop), if the workspace holds them
        if (nsuper >= 32u && tiles < 2ull * num_cus && 2ull * m * n <= kGemmPartFloats) {
            // or the next tile up in two splits as one round with a deeper
            // pipeline (8B down at M = 512: 128x128 in two splits, 3 stages,
            // 35.5 us against 48-50 for 64x128 in two before the pipelined
            // loop; since, alone, 29-33 us against 28 for 64x128 unsplit with
            // 4 stages, but inside the config-5 stack's layer sequence the
            // split plan stays ahead)
            const GemmTile &u = kGemmTiles[2];
            const uint64_t tu = (uint64_t)ceil_div(m, u.bm) * ceil_div(n, u.bn);
            if (pick == 3 && (uint64_t)ceil_div(m, u.bm) * u.bm * 4u <= (uint64_t)m * 5u && 2u * tu <= num_cus &&
                8u * 2u * tu >= 7ull * num_cus)
                return {2, 2u};
            return {pick, 2u};
        }
        return {pick, 1u};
    }
    // short K over at least half the CUs: no split either (its partial sums
    // cost more than the idle CUs: 6144x4096 at M = 128, 192 tiles of 32x128,
    // 8.2 vs 11.1 us split in two; 4096x4096 at M = 128, 128 tiles, 8.0 vs
    // 9.9; 8B gate|up at M = 32, 224 tiles, 17.0 vs 19.7)
    if (nsuper < 32u && 2u * tiles >= num_cus) return {pick, 1u};
    if (tiles * 8u >= 7ull * num_cus) return {pick, 1u};
    // steps per split: as few as reach one workgroup per CU; kz = ceil(nsuper / per) leaves no split empty
    uint32_t per = std::max<uint32_t>(1u, nsuper / ceil_div(num_cus, tiles));
    uint32_t kz = ceil_div(nsuper, per);
    while (kz > 1 && (uint64_t)kz * m * n > kGemmPartFloats) kz = ceil_div(nsuper, ++per);
    return {pick, kz};
}

// The tile and K split, then the K pipeline: where the grid is one round of
// one workgroup per CU (tiles x splits <= CUs), the deepest compiled one;
// else double buffering (a deeper ring leaves fewer workgroups per CU).
// Measured at M = 512 (us, 2 / 3 / 4 stages): 4096x4096 64x128 17.5 / 14.4
// / 13.9; 1024x4096 32x128 in two splits 12.2 / - / 10.9; 6144x4096 64x128
// (384 tiles) 19.6 / 21.4 / 24.6; 14336x4096 128x128 (448 tiles) 36.2 /
// 39.5; 4096x14336 128x128 in two splits 45.3 / 35.5.  Same MFMA sequence at
// any depth: bit-identical outputs.
GemmPlan gemm_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t num_cus)
{
    GemmPlan p = gemm_plan_tile(m, n, k, num_cus);
    if (p.tile == kGemmSkinny) return p;
    const uint64_t grid = (uint64_t)ceil_div(m, kGemmTiles[p.tile].bm) * ceil_div(n, kGemmTiles[p.tile].bn) * p.kz;
    p.nst = grid <= num_cus ? gemm_deep_stages(p.tile) : 2;
    if (t_gemm_stages) p.nst = t_gemm_stages;
    return p;
}

// The 8-wave ping-pong kernel (rfp4_gemm_<tile>_pp) for a plan of the
// 256x256 or 256x128 tile: compiled for those two, and its DMA sources are
// 32-bit offsets from the matrix bases, so each matrix's codes stay under
// 4 GiB.
bool gemm_use_pp(const GemmPlan &p, uint32_t m, uint32_t n, uint32_t k)
{
    if (p.tile != 0 && p.tile != 1) return false;
    if ((uint64_t)m * k / 2u >= (1ull << 32) || (uint64_t)n * k / 2u >= (1ull << 32)) return false;
    if (t_gemm_pp) return t_gemm_pp == 2;
    return p.tile == 0; // 256x256 (M = 512: gate|up 47.0 -> 43.2 us, LM head 208.9 -> 193.6 us); 256x128 is slower
}

} // namespace

extern "C" {

int fp4_gemm(rfp4_stream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes,
             const uint8_t *a_scales, const uint8_t *w_codes, const uint8_t *w_scales, float *c)
{
    return gemm_launch((hipStream_t)stream, m, n, k, a_codes, a_scales, nullptr, w_codes, w_scales, nullptr, c,
                       g_rt ? g_rt->gemm_part : nullptr);
}

int fp4_gemm_tiled(rfp4_stream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes,
                   const uint8_t *a_scales, const uint8_t *a_scales_tiled, const uint8_t *w_codes,
                   const uint8_t *w_scales, const uint8_t *w_scales_tiled, float *c)
{
    if (!a_scales_tiled || !w_scales_tiled) return set_error(RFP4_E_INVALID, "fp4_gemm_tiled: null step-blocked scales");
    if (((uintptr_t)a_scales_tiled | (uintptr_t)w_scales_tiled) & 3u)
        return set_error(RFP4_E_ALIGN, "fp4_gemm_tiled: step-blocked scales must be 4-byte aligned");
    return gemm_launch((hipStream_t)stream, m, n, k, a_codes, a_scales, a_scales_tiled, w_codes, w_scales,
                       w_scales_tiled, c, g_rt ? g_rt->gemm_part : nullptr);
}

} // extern "C"

namespace rfp4 {

// Where the plan's kernel has the accumulating epilogue: the tiled kernels
// but the 4-wave 256x256 one (the ping-pong 256x256 kernel has it).
bool gemm_accumulate_ok(uint32_t m, uint32_t n, uint32_t k)
{
    Runtime *rt = g_rt;
    if (!rt || !m || !n || !k || k % 256u) return false;
    const GemmPlan p = gemm_plan(m, n, k, (uint32_t)rt->num_cus);
    return p.tile != kGemmSkinny && (p.tile != 0 || gemm_use_pp(p, m, n, k));
}

int gemm_launch(hipStream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes, const uint8_t *a_scales,
                const uint8_t *a_st, const uint8_t *w_codes, const uint8_t *w_scales, const uint8_t *w_st, float *c,
                float *part, bool accumulate)
{
    if (!a_codes || !a_scales || !w_codes || !w_scales || !c) return set_error(RFP4_E_INVALID, "fp4_gemm: null pointer");
    if (m == 0 || n == 0 || k == 0) return set_error(RFP4_E_SHAPE, "fp4_gemm: empty shape m=%u n=%u k=%u", m, n, k);
    if (k % 256u) return set_error(RFP4_E_SHAPE, "fp4_gemm: k=%u must be a multiple of 256", k);
    if (n % 4u) return set_error(RFP4_E_SHAPE, "fp4_gemm: n=%u must be a multiple of 4", n);
    if (((uintptr_t)a_codes | (uintptr_t)w_codes | (uintptr_t)c) & 15u)
        return set_error(RFP4_E_ALIGN, "fp4_gemm: codes and c must be 16-byte aligned");
    if (((uintptr_t)a_scales | (uintptr_t)w_scales) & 7u)
        return set_error(RFP4_E_ALIGN, "fp4_gemm: scales must be 8-byte aligned");
    Runtime *rt = g_rt;
    if (!rt) return set_error(RFP4_E_NOT_INIT, "rfp4_init has not been called");
    GemmPlan p = gemm_plan(m, n, k, (uint32_t)rt->num_cus);
    if (p.tile == kGemmSkinny) {
        if (accumulate) return set_error(RFP4_E_INVALID, "fp4_gemm: no accumulating few-row kernel (m=%u)", m);
        if (!gemm_skinny_ok(m, k))
            return set_error(RFP4_E_SHAPE, "fp4_gemm: the few-row kernel needs k a multiple of 512, up to 16384 for "
                                           "m <= 32 and up to 8192 for m <= 64 (m=%u k=%u)", m, k);
        if (!gemm_rows_has(p.ma, p.nb, (int)p.kz))
            return set_error(RFP4_E_INVALID, "fp4_gemm: no few-row variant with %d W fragments for m=%u k=%u", (int)p.kz, m, k);
        char name[48];
        snprintf(name, sizeof name, "rfp4_gemm_rows_m%d_s%d_f%u", 16 * p.ma, p.nb, p.kz);
        const uint32_t waves = ceil_div(k / 512u, (uint32_t)p.nb);
        GemmArgs a{a_codes, a_scales, w_codes, w_scales, c, nullptr, m, n, k, 1u};
        return launch(name, dim3(ceil_div(n, 16u * p.kz)), dim3(64u * waves), (hipStream_t)stream, &a);
    }
    const GemmTile &t = kGemmTiles[p.tile];
    const uint64_t tiles = (uint64_t)ceil_div(m, t.bm) * ceil_div(n, t.bn);
    if (p.kz > 1 && (uint64_t)p.kz * m * n > kGemmPartFloats)
        return set_error(RFP4_E_CAPACITY, "fp4_gemm: split-K partials %u x %u x %u exceed the workspace", p.kz, m, n);
    if (tiles * p.kz > 0x7FFFFFFFull) return set_error(RFP4_E_SHAPE, "fp4_gemm: grid too large");
    if (p.kz > 1 && !part) return set_error(RFP4_E_INVALID, "fp4_gemm: split-K plan without a workspace");
    if (!a_st || !w_st) {
        // the step-blocked scale copies the tiled kernels read, made here (stream-ordered before the GEMM)
        const size_t abytes = (scales_tiled_bytes(m, k) + 255u) / 256u * 256u, wbytes = scales_tiled_bytes(n, k);
        if (abytes + wbytes > kGemmStBytes)
            return set_error(RFP4_E_CAPACITY, "fp4_gemm: step-blocked scales of %u + %u rows x k=%u exceed the %zu-byte "
                                              "workspace (pass them to fp4_gemm_tiled)", m, n, k, kGemmStBytes);
        uint8_t *ast = rt->gemm_st, *wst = rt->gemm_st + abytes;
        const int rc = scales_tile_launch(stream, k, a_scales, ast, m, w_scales, wst, n);
        if (rc) return rc;
        a_st = ast;
        w_st = wst;
    }
    // two-way splits sum in the launch (the last split of a tile to arrive),
    // others in the reduce kernel launched next (also tiles above 256x128,
    // whose kernels have no registers for the other plane, and the ping-pong
    // kernels)
    const bool pp = gemm_use_pp(p, m, n, k);
    if (accumulate && p.tile == 0 && !pp)
        return set_error(RFP4_E_INVALID, "fp4_gemm: no accumulating 4-wave 256x256 kernel (the ping-pong one has it)");
    uint32_t *counters = p.kz == 2u && t.bm * t.bn <= 256u * 128u && tiles <= kGemmCounters && !t_gemm_reduce_kernel && !pp
                             ? (uint32_t *)(part + kGemmPartFloats) : nullptr;
    GemmArgs a{a_codes, a_scales, w_codes, w_scales, c, part, m, n, k, p.kz, counters, a_st, w_st};
    a.c_add = accumulate ? 1u : 0u;
    char pname[48];
    const char *kname = t.name;
    if (pp) { // 8 waves, two per SIMD (kernels.hip GEMM_KERNEL_PP)
        snprintf(pname, sizeof pname, "%s_pp", t.name);
        kname = pname;
    } else if (p.nst >= 3) { // a deeper DMA pipeline (kernels.hip GEMM_KERNEL_P)
        snprintf(pname, sizeof pname, "%s_p%d", t.name, p.nst);
        kname = pname;
    }
    int rc = launch(kname, dim3((unsigned)(tiles * p.kz)), dim3(pp ? 512 : 256), (hipStream_t)stream, &a);
    if (rc || p.kz == 1 || counters) return rc;
    const uint64_t n4 = (uint64_t)m * n / 4u;
    return launch("rfp4_gemm_reduce", dim3((unsigned)std::min<uint64_t>((n4 + 255u) / 256u, 8192u)), dim3(256),
                  (hipStream_t)stream, &a);
}

// The kernel with the SwiGLU epilogue for the plan of the plain GEMM (m, 2
// ffn, k), no K split: the 256x256 ping-pong tile (ffn % 256 == 0: whole
// 128-column pairs and step-blocked output scales), or the 128x128 tile with
// 2 or 3 stages (64-column pairs).  Null: none.
static const char *gemm_swiglu_kernel(uint32_t m, uint32_t ffn, uint32_t k, uint32_t &cols)
{
    Runtime *rt = g_rt;
    if (!rt || m == 0 || ffn == 0 || ffn % 256u || k == 0 || k % 256u) return nullptr;
    const GemmPlan p = gemm_plan(m, 2u * ffn, k, (uint32_t)rt->num_cus);
    if (p.kz != 1u) return nullptr;
    const bool pp = gemm_use_pp(p, m, 2u * ffn, k);
    if (p.tile == 0 && pp) {
        cols = 128u;
        return "rfp4_gemm_256x256_ppsw";
    }
    if (p.tile == 2 && !pp && (p.nst == 2 || p.nst == 3)) {
        cols = 64u;
        return p.nst == 2 ? "rfp4_gemm_128x128_sw" : "rfp4_gemm_128x128_p3_sw";
    }
    return nullptr;
}

bool gemm_swiglu_ok(uint32_t m, uint32_t ffn, uint32_t k)
{
    uint32_t cols = 0;
    return gemm_swiglu_kernel(m, ffn, k, cols) != nullptr;
}

int gemm_swiglu_launch(hipStream_t stream, uint32_t m, uint32_t ffn, uint32_t k, const uint8_t *a_codes,
                       const uint8_t *a_scales, const uint8_t *a_st, const uint8_t *w_codes, const uint8_t *w_scales,
                       const uint8_t *w_st, uint8_t *q_codes, uint8_t *q_scales, uint8_t *q_scales_t)
{
    if (!a_codes || !a_st || !w_codes || !w_st || !q_codes || !q_scales)
        return set_error(RFP4_E_INVALID, "gemm_swiglu: null pointer");
    if (((uintptr_t)a_codes | (uintptr_t)w_codes) & 15u || ((uintptr_t)q_codes | (uintptr_t)a_st | (uintptr_t)w_st) & 3u)
        return set_error(RFP4_E_ALIGN, "gemm_swiglu: misaligned codes or scales");
    uint32_t cols = 0;
    const char *kname = gemm_swiglu_kernel(m, ffn, k, cols);
    if (!kname)
        return set_error(RFP4_E_SHAPE, "gemm_swiglu: the plan of %u x %u x %u has no SwiGLU epilogue", m, 2u * ffn, k);
    GemmArgs a{a_codes, a_scales, w_codes, w_scales, nullptr, nullptr, m, 2u * ffn, k, 1u, nullptr, a_st, w_st,
               q_codes, q_scales, q_scales_t, ffn, 0u};
    const uint32_t bm = cols == 128u ? 256u : 128u; // tile rows
    const uint64_t tiles = (uint64_t)((m + bm - 1u) / bm) * (ffn / cols);
    return launch(kname, dim3((unsigned)tiles), dim3(cols == 128u ? 512 : 256), stream, &a);
}

// The _rope kernel for the plan of (m, n, k), no K split: the plan's
// 4-wave kernel with the epilogue (kernels.hip GEMM_KERNEL_ROPE /
// GEMM_KERNEL_P_ROPE: the tiles up to 128 rows, at the stage counts the
// planner uses), or the ping-pong 256x256 one (false: none).
struct RopeKernel {
    char name[48];
    int tile;
    unsigned threads;
};
static bool gemm_rope_kernel(uint32_t m, uint32_t n, uint32_t k, RopeKernel &rk)
{
    Runtime *rt = g_rt;
    if (!rt || m == 0 || n == 0 || k == 0 || k % 256u) return false;
    const GemmPlan p = gemm_plan(m, n, k, (uint32_t)rt->num_cus);
    if (p.tile == kGemmSkinny || p.kz != 1u) return false;
    const bool pp = gemm_use_pp(p, m, n, k);
    rk.tile = p.tile;
    if (p.tile == 0) {
        if (!pp) return false;
        snprintf(rk.name, sizeof rk.name, "rfp4_gemm_256x256_pp_rope");
        rk.threads = 512u;
        return true;
    }
    if (pp) return false;
    // compiled: 128x128, 64x128 and 32x128 with 2 stages; 3 for 64x128 and
    // 128x128; 4 for 32x128 and 64x128 (no 256x128: slower than the GEMM +
    // the row kernel where measured)
    const int nst = p.nst;
    const bool ok = p.tile >= 2 && (nst == 2 || (nst == 3 && (p.tile == 2 || p.tile == 3)) ||
                                    (nst == 4 && (p.tile == 3 || p.tile == 4)));
    if (!ok) return false;
    if (nst == 2) snprintf(rk.name, sizeof rk.name, "%s_rope", kGemmTiles[p.tile].name);
    else snprintf(rk.name, sizeof rk.name, "%s_p%d_rope", kGemmTiles[p.tile].name, nst);
    rk.threads = 256u;
    return true;
}

bool gemm_rope_ok(uint32_t m, uint32_t n, uint32_t k, uint32_t hd)
{
    RopeKernel rk;
    if (!(hd == 64u || hd == 128u) || n % hd || !gemm_rope_kernel(m, n, k, rk)) return false;
    // a head lies in one column tile (the tile widths are multiples of 128)
    return kGemmTiles[rk.tile].bn % hd == 0u;
}

int gemm_rope_launch(hipStream_t stream, uint32_t m, uint32_t n, uint32_t k, const uint8_t *a_codes,
                     const uint8_t *a_scales, const uint8_t *a_st, const uint8_t *w_codes, const uint8_t *w_scales,
                     const uint8_t *w_st, float *c, const GemmRope &r)
{
    if (!a_codes || !a_st || !w_codes || !w_st || !c || !r.cosv || !r.sinv || !r.kc || !r.vc)
        return set_error(RFP4_E_INVALID, "gemm_rope: null pointer");
    if (((uintptr_t)a_codes | (uintptr_t)w_codes | (uintptr_t)c) & 15u || ((uintptr_t)a_st | (uintptr_t)w_st) & 3u)
        return set_error(RFP4_E_ALIGN, "gemm_rope: misaligned codes, scales or output");
    if (!gemm_rope_ok(m, n, k, r.hd) || r.q % r.hd || r.kv % r.hd || n != r.q + 2u * r.kv)
        return set_error(RFP4_E_SHAPE, "gemm_rope: no RoPE epilogue for %u x %u x %u with heads of %u (q %u, kv %u)", m,
                         n, k, r.hd, r.q, r.kv);
    RopeKernel rk;
    gemm_rope_kernel(m, n, k, rk);
    const GemmTile &t = kGemmTiles[rk.tile];
    GemmArgs a{a_codes, a_scales, w_codes, w_scales, c, nullptr, m, n, k, 1u, nullptr, a_st, w_st,
               nullptr, nullptr, nullptr, 0u, 0u, r.cosv, r.sinv, r.kc, r.vc, r.ts, r.hs, r.pos0, r.q, r.kv, r.hd};
    const uint64_t tiles = (uint64_t)ceil_div(m, t.bm) * ceil_div(n, t.bn);
    return launch(rk.name, dim3((unsigned)tiles), dim3(rk.threads), stream, &a);
}

} // namespace rfp4

extern "C" {

int rfp4_debug_attn_chunk(uint32_t chunk)
{
    t_force_attn_chunk = chunk;
    return RFP4_OK;
}

int rfp4_debug_gemm_reduce_kernel(int on)
{
    if (on != 0 && on != 1) return set_error(RFP4_E_INVALID, "GEMM reduce mode must be 0 (auto) or 1 (reduce kernel)");
    t_gemm_reduce_kernel = on;
    return RFP4_OK;
}

int rfp4_debug_gemm_stages(int nst)
{
    if (nst != 0 && (nst < 2 || nst > 4)) return set_error(RFP4_E_INVALID, "GEMM stages must be 0 (auto), 2, 3 or 4");
    t_gemm_stages = nst;
    return RFP4_OK;
}

int rfp4_debug_gemm_pp(int mode)
{
    if (mode < 0 || mode > 2) return set_error(RFP4_E_INVALID, "GEMM ping-pong mode must be 0 (auto), 1 (off) or 2 (on)");
    t_gemm_pp = mode;
    return RFP4_OK;
}

int rfp4_debug_gemm_plan(int tile, int kz)
{
    if (tile < -1 || tile > kGemmSkinny) return set_error(RFP4_E_INVALID, "tile must be -1 (auto) or 0..%d", kGemmSkinny);
    if (kz < 0) return set_error(RFP4_E_INVALID, "kz must be 0 (auto) or positive");
    t_gemm_tile = tile;
    t_gemm_kz = kz;
    return RFP4_OK;
}

int rfp4_gemm_plan(uint32_t m, uint32_t n, uint32_t k, int *tile_m, int *tile_n, int *kz)
{
    Runtime *rt = g_rt;
    const uint32_t cus = rt ? (uint32_t)rt->num_cus : 256u;
    if (k == 0 || k % 256u || m == 0 || n == 0) return set_error(RFP4_E_SHAPE, "gemm_plan: bad shape");
    GemmPlan p = gemm_plan(m, n, k, cus);
    const GemmTile *t = p.tile == kGemmSkinny ? nullptr : &kGemmTiles[p.tile];
    if (tile_m) *tile_m = t ? (int)t->bm : 16 * p.ma;
    if (tile_n) *tile_n = t ? (int)t->bn : 16 * (int)p.kz;
    if (kz) *kz = (int)p.kz;
    return RFP4_OK;
}

int rfp4_gemm_plan_kernel(uint32_t m, uint32_t n, uint32_t k, char *buf, size_t cap)
{
    Runtime *rt = g_rt;
    const uint32_t cus = rt ? (uint32_t)rt->num_cus : 256u;
    if (!buf || cap == 0) return set_error(RFP4_E_INVALID, "gemm_plan_kernel: null buffer");
    if (k == 0 || k % 256u || m == 0 || n == 0) return set_error(RFP4_E_SHAPE, "gemm_plan_kernel: bad shape");
    GemmPlan p = gemm_plan(m, n, k, cus);
    char name[64];
    if (p.tile == kGemmSkinny)
        snprintf(name, sizeof name, "rfp4_gemm_rows_m%d_s%d_f%u", 16 * p.ma, p.nb, p.kz);
    else if (gemm_use_pp(p, m, n, k))
        snprintf(name, sizeof name, "%s_pp/kz%u", kGemmTiles[p.tile].name, p.kz);
    else if (p.nst >= 3)
        snprintf(name, sizeof name, "%s_p%d/kz%u", kGemmTiles[p.tile].name, p.nst, p.kz);
    else
        snprintf(name, sizeof name, "%s/kz%u", kGemmTiles[p.tile].name, p.kz);
    if (strlen(name) + 1 > cap) return set_error(RFP4_E_CAPACITY, "gemm_plan_kernel: %zu bytes needed", strlen(name) + 1);
    memcpy(buf, name, strlen(name) + 1);
    return RFP4_OK;
}


int rfp4_mma_tile16(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, const uint32_t *sa,
                    const uint32_t *sb, float *out)
{
    if (!a || !b || !sa || !sb || !out) return set_error(RFP4_E_INVALID, "mma_tile16: null pointer");
    MmaTileArgs args{a, b, sa, sb, out, 0, 0};
    return launch("rfp4_mma16_tile", dim3(1), dim3(64), (hipStream_t)stream, &args);
}

int rfp4_mma_tile32(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, const uint32_t *sa,
                    const uint32_t *sb, float *out)
{
    if (!a || !b || !sa || !sb || !out) return set_error(RFP4_E_INVALID, "mma_tile32: null pointer");
    MmaTileArgs args{a, b, sa, sb, out, 0, 0};
    return launch("rfp4_mma32_tile", dim3(1), dim3(64), (hipStream_t)stream, &args);
}

int rfp4_selftest_cvt_fp4(rfp4_stream_t stream, uint32_t n, const uint32_t *words, float *out)
{
    if (!words || !out) return set_error(RFP4_E_INVALID, "selftest_cvt: null pointer");
    SelftestArgs a{words, out, nullptr, n, 0};
    return launch("rfp4_selftest_cvt", dim3((n + 255) / 256), dim3(256), (hipStream_t)stream, &a);
}

int rfp4_mma_bf16_tile(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, float *out)
{
    if (!a || !b || !out) return set_error(RFP4_E_INVALID, "mma_bf16_tile: null pointer");
    MmaTileArgs args{a, b, nullptr, nullptr, out, 0, 0};
    return launch("rfp4_mma_bf16_tile", dim3(1), dim3(64), (hipStream_t)stream, &args);
}

int rfp4_mma_f16_tile(rfp4_stream_t stream, const uint32_t *a, const uint32_t *b, float *out)
{
    if (!a || !b || !out) return set_error(RFP4_E_INVALID, "mma_f16_tile: null pointer");
    MmaTileArgs args{a, b, nullptr, nullptr, out, 1, 0};
    return launch("rfp4_mma_bf16_tile", dim3(1), dim3(64), (hipStream_t)stream, &args);
}

int rfp4_synth_mx_weight(rfp4_stream_t stream, uint64_t seed, uint64_t stream_id, float sigma, uint64_t k, uint64_t r0,
                         uint64_t nrows, uint8_t *codes, uint8_t *scales)
{
    if (!codes || !scales) return set_error(RFP4_E_INVALID, "synth_mx_weight: null pointer");
    if (k == 0 || k % 32) return set_error(RFP4_E_SHAPE, "synth_mx_weight: k not a multiple of 32");
    if (((uintptr_t)codes & 15u) != 0) return set_error(RFP4_E_ALIGN, "synth_mx_weight: codes must be 16-byte aligned");
    SynthWeightArgs a{codes, scales, seed, stream_id, r0, nrows, k, ih4_coef(sigma), 0};
    uint64_t blocks = (nrows * (k / 32) + 255) / 256;
    if (blocks > 262144) blocks = 262144;
    return launch("rfp4_synth_weight", dim3((unsigned)blocks), dim3(256), (hipStream_t)stream, &a);
}

int rfp4_synth_f16(rfp4_stream_t stream, uint64_t seed, uint64_t stream_id, float sigma, float offset, uint64_t n,
                   uint16_t *out)
{
    if (!out) return set_error(RFP4_E_INVALID, "synth_f16: null pointer");
    SynthF16Args a{out, seed, stream_id, n, ih4_coef(sigma), offset};
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 262144) blocks = 262144;
    return launch("rfp4_synth_f16", dim3((unsigned)blocks), dim3(256), (hipStream_t)stream, &a);
}

} // extern "C"
