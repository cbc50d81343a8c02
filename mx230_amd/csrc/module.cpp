// The gfx950 code object of libmxfa: checked and loaded per device with
// hipModuleLoadData, its kernels found by name (fa_kernels.h) and launched
// with hipModuleLaunchKernel. The host library holds no device code.
//
// This replaces the reference's module handling: PTX built by build.rs
// (kernel-build/src/lib.rs:37-55, :89-115), loaded with load_ptx and looked
// up by function name (02-flash-attention/src/main.rs:392-415), including
// load_ptx's guard against an empty stub module (common/src/lib.rs:11-18):
// here a missing or malformed code object is an MXFA_ERR_CODE_OBJECT status.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iterator>
#include <mutex>
#include <string>
#include <vector>

#include "fa_kernels.h"
#include "fa_launch.h"

namespace mxfa {

namespace {

const char *const kNames[kNumKernels] = {
#define MXFA_KNAME(n) #n,
    MXFA_KERNEL_LIST(MXFA_KNAME)
#undef MXFA_KNAME
};

constexpr int kMaxDevices = 64;
constexpr const char *kCodeObjectFile = "mxfa_gfx950.hsaco";

struct DeviceModule {
    std::atomic<bool> ready{false};
    hipModule_t mod = nullptr;
    hipFunction_t fn[kNumKernels] = {};
    void *fallbacks = nullptr;  // the code object's Delta fallback counter
    void *timeouts = nullptr;   // and its reduce timeout counter
    int cus = 0;                // the device's CUs
    // work-groups of 256 threads of each kernel resident per CU (-1: not asked yet)
    std::atomic<int> occupancy[kNumKernels];
    DeviceModule() {
        for (auto &o : occupancy) o.store(-1);
    }
};

std::mutex g_mu;
DeviceModule g_dev[kMaxDevices];
std::string g_path;  // empty: kCodeObjectFile beside libmxfa.so

std::string default_path() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void *>(&default_path), &info) != 0 && info.dli_fname != nullptr) {
        std::string lib(info.dli_fname);
        const size_t slash = lib.rfind('/');
        if (slash != std::string::npos) return lib.substr(0, slash + 1) + kCodeObjectFile;
    }
    return kCodeObjectFile;
}

std::string current_path() {
    std::lock_guard<std::mutex> lock(g_mu);
    return g_path.empty() ? default_path() : g_path;
}

uint16_t rd16(const std::vector<char> &b, size_t o) {
    return (uint16_t)((unsigned char)b[o] | ((unsigned char)b[o + 1] << 8));
}
uint32_t rd32(const std::vector<char> &b, size_t o) { return (uint32_t)rd16(b, o) | ((uint32_t)rd16(b, o + 2) << 16); }

// Reads a code object and checks its ELF header: 64-bit little-endian ELF,
// machine EM_AMDGPU (224), OS/ABI AMDGPU_HSA (64), processor gfx950
// (EF_AMDGPU_MACH, the low byte of e_flags, 0x4f).
CodeObjectStatus read_code_object(const std::string &path, std::vector<char> &bytes) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return CodeObjectStatus::kMissing;
    bytes.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    if (bytes.size() < 64) return CodeObjectStatus::kInvalid;
    if (std::memcmp(bytes.data(), "\x7f" "ELF", 4) != 0) return CodeObjectStatus::kInvalid;
    if (bytes[4] != 2 || bytes[5] != 1) return CodeObjectStatus::kInvalid;  // ELFCLASS64, little-endian
    if ((unsigned char)bytes[7] != 64) return CodeObjectStatus::kInvalid;    // ELFOSABI_AMDGPU_HSA
    if (rd16(bytes, 18) != 224) return CodeObjectStatus::kInvalid;           // EM_AMDGPU
    if ((rd32(bytes, 48) & 0xffu) != 0x4fu) return CodeObjectStatus::kWrongArch;  // gfx950
    return CodeObjectStatus::kOk;
}

void unload(DeviceModule &m) {
    if (m.mod != nullptr) (void)hipModuleUnload(m.mod);
    m.mod = nullptr;
    m.fallbacks = nullptr;
    m.timeouts = nullptr;
    std::memset(m.fn, 0, sizeof(m.fn));
    for (auto &o : m.occupancy) o.store(-1);
    m.cus = 0;
    m.ready.store(false);
}

// The module of `device` (current on the calling thread), loaded on first use.
DeviceModule *module_for(int device, hipError_t *err) {
    if (device < 0 || device >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    DeviceModule &m = g_dev[device];
    if (m.ready.load(std::memory_order_acquire)) return &m;
    std::lock_guard<std::mutex> lock(g_mu);
    if (m.ready.load(std::memory_order_relaxed)) return &m;
    std::vector<char> bytes;
    const std::string path = g_path.empty() ? default_path() : g_path;
    if (read_code_object(path, bytes) != CodeObjectStatus::kOk) {
        *err = hipErrorInvalidImage;
        return nullptr;
    }
    // failed runtime calls below are reported as hipErrorInvalidImage (the
    // caller's status); the runtime's own record of them is cleared, so the
    // caller's next runtime call does not report it again
    if (hipModuleLoadData(&m.mod, bytes.data()) != hipSuccess) {
        (void)hipGetLastError();
        m.mod = nullptr;
        *err = hipErrorInvalidImage;
        return nullptr;
    }
    for (int i = 0; i < kNumKernels; ++i) {
        if (hipModuleGetFunction(&m.fn[i], m.mod, kNames[i]) != hipSuccess) {
            (void)hipGetLastError();
            unload(m);
            *err = hipErrorInvalidImage;
            return nullptr;
        }
    }
    hipDeviceptr_t ptr = nullptr;
    size_t bytes_g = 0;
    if (hipModuleGetGlobal(&ptr, &bytes_g, m.mod, "mxfa_delta_fallbacks") != hipSuccess ||
        bytes_g != sizeof(unsigned long long)) {
        (void)hipGetLastError();
        unload(m);
        *err = hipErrorInvalidImage;
        return nullptr;
    }
    m.fallbacks = ptr;
    if (hipModuleGetGlobal(&ptr, &bytes_g, m.mod, "mxfa_reduce_timeouts") != hipSuccess ||
        bytes_g != sizeof(unsigned long long)) {
        (void)hipGetLastError();
        unload(m);
        *err = hipErrorInvalidImage;
        return nullptr;
    }
    m.timeouts = ptr;
    if (hipDeviceGetAttribute(&m.cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
        (void)hipGetLastError();
        m.cus = 0;
    }
    m.ready.store(true, std::memory_order_release);
    return &m;
}

DeviceModule *current_module(hipError_t *err) {
    int device = -1;
    const hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    return module_for(device, err);
}

}  // namespace

CodeObjectStatus check_code_object(const char *path) {
    std::vector<char> bytes;
    return read_code_object(path != nullptr ? std::string(path) : current_path(), bytes);
}

void set_code_object_path(const char *path) {
    std::lock_guard<std::mutex> lock(g_mu);
    g_path = path != nullptr ? std::string(path) : std::string();
}

hipError_t load_code_object(int device) {
    hipError_t err = hipSuccess;
    return module_for(device, &err) != nullptr ? hipSuccess : err;
}

void unload_code_objects() {
    int current = -1;
    const bool restore = hipGetDevice(&current) == hipSuccess;
    std::lock_guard<std::mutex> lock(g_mu);
    for (int d = 0; d < kMaxDevices; ++d) {
        if (g_dev[d].mod == nullptr) continue;
        if (hipSetDevice(d) == hipSuccess) unload(g_dev[d]);
    }
    if (restore) (void)hipSetDevice(current);
}

int device_cus() {
    hipError_t err = hipSuccess;
    DeviceModule *m = current_module(&err);
    return m == nullptr ? 0 : m->cus;
}

int kernel_occupancy(KernelId id) {
    hipError_t err = hipSuccess;
    DeviceModule *m = current_module(&err);
    if (m == nullptr) return 0;
    int n = m->occupancy[id].load();
    if (n < 0) {
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, m->fn[id], 256, 0) != hipSuccess) {
            (void)hipGetLastError();
            n = 0;
        }
        m->occupancy[id].store(n);
    }
    return n;
}

void cu_balance(Params *p, KernelId id, long long groups) {
    constexpr int kXcds = 8;  // MI355X: 8 XCDs of 32 CUs
    p->cu_run = p->cu_runs = 0;
    const int cus = device_cus();
    if (cus <= 0 || cus % kXcds != 0) return;
    const int occ = kernel_occupancy(id);
    if (occ <= 0) return;
    const long long resident = std::min(groups, (long long)cus * occ);
    const long long runs = resident / cus;
    // launches of more than 1.5 rounds of resident work-groups keep their
    // order: their later rounds, handed out heaviest first as slots free up,
    // balance the CUs already (A/B, forward, median of 6, us: north star 109.9
    // plain against 111.5 reordered, B4 H12 N4000 108.0 against 110.4; cfg4,
    // 1.17 rounds, 70.1 against 67.0)
    if (runs < 2 || 2 * groups > 3 * resident) return;
    p->cu_run = cus;
    p->cu_runs = (int)runs;
}

hipError_t launch_kernel(KernelId id, dim3 grid, dim3 block, void **args, hipStream_t stream) {
    hipError_t err = hipSuccess;
    DeviceModule *m = current_module(&err);
    if (m == nullptr) return err;
    return hipModuleLaunchKernel(m->fn[id], grid.x, grid.y, grid.z, block.x, block.y, block.z, 0, stream, args,
                                 nullptr);
}

hipError_t read_wg_times(void *dst, size_t bytes, size_t *avail) {
    hipError_t err = hipSuccess;
    DeviceModule *m = current_module(&err);
    if (m == nullptr) return err;
    hipDeviceptr_t ptr = nullptr;
    size_t n = 0;
    // present only in the timeline build of the code object; the runtime's
    // record of the failed lookup is cleared, the status reports it
    if (hipModuleGetGlobal(&ptr, &n, m->mod, "mxfa_wg_times") != hipSuccess) {
        (void)hipGetLastError();
        return hipErrorNotFound;
    }
    *avail = n;
    if (dst == nullptr || bytes == 0) return hipSuccess;
    return hipMemcpyDtoH(dst, ptr, bytes < n ? bytes : n);
}

hipError_t read_delta_fallbacks(unsigned long long *count) {
    hipError_t err = hipSuccess;
    DeviceModule *m = current_module(&err);
    if (m == nullptr) return err;
    return hipMemcpyDtoH(count, m->fallbacks, sizeof(*count));
}

hipError_t read_reduce_timeouts(unsigned long long *count) {
    hipError_t err = hipSuccess;
    DeviceModule *m = current_module(&err);
    if (m == nullptr) return err;
    return hipMemcpyDtoH(count, m->timeouts, sizeof(*count));
}

}  // namespace mxfa
