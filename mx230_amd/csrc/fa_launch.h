// Host-side launchers of the flash-attention kernels (internal to libmxfa).
// Each returns hipSuccess or the launch error; shapes are validated by the
// C ABI (mxfa_api.cpp) before any of these is called.
#pragma once

#include <hip/hip_runtime.h>

#include "fa_device.h"
#include "fa_kernels.h"

namespace mxfa {

// ---- the scratch of mxfa_run_bwd_noalloc (scratch.hip): a static device array
size_t noalloc_scratch_bytes();
// its device address on `device` (current on the calling thread)
hipError_t noalloc_scratch(int device, void **ptr);

// ---- the code object (module.cpp)
enum class CodeObjectStatus { kOk, kMissing, kInvalid, kWrongArch };
// Host-side check of a code object file (the current path when NULL): no
// device access.
CodeObjectStatus check_code_object(const char *path);
// The code object later loads read (NULL: mxfa_gfx950.hsaco beside libmxfa.so).
void set_code_object_path(const char *path);
// Loads the code object on `device` (current on the calling thread) if it is
// not loaded yet; hipErrorInvalidImage if it is missing, malformed or lacks
// a kernel.
hipError_t load_code_object(int device);
// Unloads every device's code object (the next launch loads it again).
void unload_code_objects();
// Launches kernel `id` of the current device's code object (loading it on
// first use). args: pointers to the kernel's arguments, in order.
hipError_t launch_kernel(KernelId id, dim3 grid, dim3 block, void **args, hipStream_t stream);
// The current device's CUs, and the 256-thread work-groups of kernel `id`
// resident at once per CU (the runtime's occupancy); 0 when unknown.
int device_cus();
int kernel_occupancy(KernelId id);
// Sets p->cu_run and p->cu_runs (cu_order_wg, fa_device.h) for a causal
// launch of `groups` work-groups of kernel `id`: the device's CUs, and the
// whole runs of them among the work-groups resident at once (the CUs times
// the kernel's occupancy); no reordering where the CUs are not a multiple of
// the 8 XCDs, fewer than two runs are resident, or the launch holds more than
// 1.5 times the resident work-groups.
void cu_balance(Params *p, KernelId id, long long groups);

hipError_t launch_fwd(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream);
// The causal forward with its keys split over work-groups (grid.z) and a
// merging launch: the split count for a shape (1: no split pays), the fp32
// partials it needs in p.fwd_part, and the two launches (2 <= splits <=
// kFwdMaxSplits = 32; K/V contiguous, or through p.block_table).
int fwd_splits(const Params &p, int dtype_bf16, int d);
size_t fwd_split_workspace_bytes(const Params &p, int d, int splits);
hipError_t launch_fwd_split(const Params &p, int dtype_bf16, int d, int splits, hipStream_t stream);
hipError_t launch_preprocess(const Params &p, int dtype_bf16, int d, hipStream_t stream);
// delta != 0: the dQ pass computes Delta from p.o_in and writes it to p.delta
hipError_t launch_bwd_dq(const Params &p, int dtype_bf16, int d, int causal, int delta, hipStream_t stream);
// p.dkv_ws != nullptr: GQA shapes may split each key block's query heads'
// stages over several work-groups, with fp32 partials in p.dkv_ws (2 *
// dkv_split(p, ...) * B * Hkv * N * d floats) and a second, reducing launch
hipError_t launch_bwd_dkv(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream);
// partial planes of the split (the most shares of any key block; 1: none)
int dkv_split(const Params &p, int dtype_bf16, int d, int causal);
// the workspace the split takes (0: no split): 2 * dkv_split(...) * B * Hkv *
// N * d floats of partial planes, then 8 bytes per share for the one-launch
// backward's share flags
size_t dkv_workspace_bytes(const Params &p, int dtype_bf16, int d, int causal);
// The one-launch backward from O (dQ pass with Delta + dK/dV pass, bf16;
// with p.dkv_ws a GQA split as launch_bwd_dkv, whose reduce runs in the same
// launch, or as a second launch where the share flags do not fit): available
// for the shape, and launched with its own epoch.
bool bwd_fused_available(const Params &p, int dtype_bf16, int d, hipStream_t stream);
hipError_t launch_bwd_fused(const Params &p, int d, int causal, hipStream_t stream);
// Process-wide settings of the one-launch backward: whether it is used where
// available, and the bound of each Delta wait in microseconds (< 0: never
// wait, always compute Delta); read at every launch.
void set_bwd_options(int one_launch, int delta_wait_us, int reduce_wait_us);
void get_bwd_options(int *one_launch, int *delta_wait_us, int *reduce_wait_us);
// Delta blocks the one-launch backward's dK/dV work-groups computed
// themselves on the current device since the library was loaded (a
// synchronous copy).
hipError_t read_delta_fallbacks(unsigned long long *count);
// Reduce work-groups of the one-launch backward's GQA split whose wait for
// their shares ran out on the current device since the library was loaded
// (a synchronous copy).
hipError_t read_reduce_timeouts(unsigned long long *count);
// Timeline build only: copies up to `bytes` of the per-work-group timestamps
// to host `dst` (none when dst is NULL) and reports their size in *avail;
// hipErrorNotFound when the loaded code object is not the timeline build.
hipError_t read_wg_times(void *dst, size_t bytes, size_t *avail);
hipError_t launch_bwd_naive(const Params &p, int d, int causal, hipStream_t stream);
hipError_t launch_naive_fwd(const Params &p, float *s, int d, int causal, hipStream_t stream);

// roofline probes (probe.hip)
int probe_sink_len();
double probe_mfma_flops(int bf16, int iters);
hipError_t launch_probe_mfma(int bf16, int iters, float *sink, hipStream_t stream);
double probe_mfma32_flops(int iters);
hipError_t launch_probe_mfma32(int iters, float *sink, hipStream_t stream);
hipError_t launch_probe_read(const void *x, size_t bytes, float *sink, hipStream_t stream);
hipError_t launch_probe_copy(const void *x, void *y, size_t bytes, hipStream_t stream);
int probe_mix_count();
double probe_mix_flops(int waves_per_simd, int iters);
hipError_t launch_probe_mix(int mix, int waves_per_simd, int iters, float *sink, hipStream_t stream);
double probe_dq_atomic_bytes(int bh, int n);
hipError_t launch_probe_dq_atomic(float *acc, int bh, int n, int atomic, hipStream_t stream);

}  // namespace mxfa
