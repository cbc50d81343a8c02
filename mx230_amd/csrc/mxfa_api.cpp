// C ABI of libmxfa (declared in include/mxfa.h): argument validation, the
// mapping of mxfa_shape onto kernel parameters, and error translation. No
// device memory is allocated and nothing synchronises here.
#include "../../include/mxfa.h"
#include "../../include/mxfa_probes.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "fa_launch.h"

namespace {

using mxfa::Params;

constexpr long long kMaxGridY = 65535;

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_shape(const mxfa_shape *s) {
    if (s == nullptr) return MXFA_ERR_NULL;
    if (s->dtype != MXFA_F32 && s->dtype != MXFA_BF16) return MXFA_ERR_DTYPE;
    if (s->B < 1 || s->Hq < 1 || s->Hkv < 1 || s->N < 1 || s->d < 1) return MXFA_ERR_SHAPE;
    if (s->Hq % s->Hkv != 0) return MXFA_ERR_SHAPE;
    if (s->causal != 0 && s->causal != 1) return MXFA_ERR_SHAPE;
    if (!(s->scale >= 0.0f) || std::isinf(s->scale)) return MXFA_ERR_SHAPE;
    // grid limits: x = B*H (32-bit), y = query/key blocks
    const long long bh = (long long)s->B * s->Hq;
    if (bh > 0x7fffffffLL) return MXFA_ERR_SHAPE;
    if (((long long)s->N + 63) / 64 > kMaxGridY) return MXFA_ERR_SHAPE;
    // every tensor (and workspace) size in bytes must be far from overflowing
    // size_t: at most 2^40 elements per tensor (no single GPU holds more)
    if ((double)bh * (double)s->N * (double)s->d > 1099511627776.0) return MXFA_ERR_SHAPE;
    if (s->d != 64 && s->d != 128) return MXFA_ERR_UNSUPPORTED;
    if (s->dtype == MXFA_F32 && s->d != 64) return MXFA_ERR_UNSUPPORTED;
    return MXFA_OK;
}

Params make_params(const mxfa_shape *s) {
    Params p;
    std::memset(&p, 0, sizeof(p));
    p.B = s->B;
    p.Hq = s->Hq;
    p.Hkv = s->Hkv;
    p.N = s->N;
    p.group = s->Hq / s->Hkv;
    p.scale = s->scale > 0.0f ? s->scale : 1.0f / std::sqrt((float)s->d);
    p.scale_log2 = p.scale * mxfa::kLog2e;
    // packed [B][H][N][d] layout, keys = queries, no causal offset
    const long long nd = (long long)s->N * s->d;
    p.q_rs = p.kv_rs = p.o_rs = s->d;
    p.q_hs = p.o_hs = p.kv_hs = nd;
    p.q_bs = p.o_bs = nd * s->Hq;
    p.kv_bs = nd * s->Hkv;
    p.Nk = s->N;
    p.pos0 = 0;
    p.block_table = nullptr;  // contiguous K/V
    p.fwd_part = nullptr;     // the unsplit forward
    p.bs_shift = 0;
    p.dkv_ws = nullptr;
    p.dkv_split = p.dkv_min_shares = 1;
    p.dkv_share_stages = 1 << 30;
    return p;
}

// hipErrorInvalidImage: the code object could not be loaded (module.cpp)
int from_hip(hipError_t e) {
    if (e == hipSuccess) return MXFA_OK;
    return e == hipErrorInvalidImage ? MXFA_ERR_CODE_OBJECT : MXFA_ERR_LAUNCH;
}

int check_ptrs(std::initializer_list<const void *> ps) {
    for (const void *p : ps) {
        if (p == nullptr) return MXFA_ERR_NULL;
    }
    for (const void *p : ps) {
        if (!aligned16(p)) return MXFA_ERR_ALIGN;
    }
    return MXFA_OK;
}

int fwd_impl(const mxfa_shape *shape, const void *q, const void *k, const void *v, void *o, float *lse,
             bool want_lse, void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = want_lse ? check_ptrs({q, k, v, o, lse}) : check_ptrs({q, k, v, o});
    if (rc != MXFA_OK) return rc;
    Params p = make_params(shape);
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.lse = want_lse ? lse : nullptr;
    return from_hip(mxfa::launch_fwd(p, shape->dtype == MXFA_BF16, shape->d, shape->causal,
                                     static_cast<hipStream_t>(stream)));
}

// A workspace is optional (NULL: the dK/dV pass reduces each GQA group in one
// work-group per key block); a given one must be 16-byte aligned and hold
// mxfa_bwd_workspace_bytes(shape).
int check_workspace(const mxfa_shape *shape, const void *ws, size_t bytes) {
    if (ws == nullptr) return MXFA_OK;
    if (!aligned16(ws)) return MXFA_ERR_ALIGN;
    return bytes < mxfa_bwd_workspace_bytes(shape) ? MXFA_ERR_WORKSPACE : MXFA_OK;
}

Params bwd_params(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *dout,
                  const float *lse, const float *delta) {
    Params p = make_params(shape);
    p.q = q;
    p.k = k;
    p.v = v;
    p.dout = dout;
    p.lse = const_cast<float *>(lse);
    p.delta = const_cast<float *>(delta);
    return p;
}

}  // namespace

extern "C" {

int mxfa_version(void) { return 100; }

const char *mxfa_strerror(int status) {
    switch (status) {
        case MXFA_OK: return "ok";
        case MXFA_ERR_NULL: return "a required pointer is NULL";
        case MXFA_ERR_SHAPE: return "invalid shape (B, Hq, Hkv, N, d, causal, scale or Hq % Hkv)";
        case MXFA_ERR_DTYPE: return "unknown dtype";
        case MXFA_ERR_UNSUPPORTED: return "no kernel for this shape (d must be 64 or 128; fp32 needs d = 64)";
        case MXFA_ERR_ALIGN: return "a device pointer is not 16-byte aligned";
        case MXFA_ERR_LAUNCH: return "the HIP runtime rejected a kernel launch";
        case MXFA_ERR_DEVICE: return "no usable gfx950 device";
        case MXFA_ERR_WORKSPACE: return "the workspace is smaller than the *_workspace_bytes(shape) of the call";
        case MXFA_ERR_SCRATCH:
            return "the shape needs more scratch than mxfa_bwd_noalloc_scratch_bytes() (use mxfa_run_bwd_ws)";
        case MXFA_ERR_CODE_OBJECT:
            return "the gfx950 code object (mxfa_gfx950.hsaco) is missing, malformed, for another processor or "
                   "lacks a kernel";
        default: return "unknown status";
    }
}

int mxfa_init(int device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return MXFA_ERR_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return MXFA_ERR_DEVICE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return MXFA_ERR_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return MXFA_ERR_DEVICE;
    if (mxfa::load_code_object(device) != hipSuccess) return MXFA_ERR_CODE_OBJECT;
    // set-up of mxfa_run_bwd_noalloc: the scratch array's address on this device
    void *scratch = nullptr;
    return mxfa::noalloc_scratch(device, &scratch) == hipSuccess ? MXFA_OK : MXFA_ERR_DEVICE;
}

int mxfa_shutdown(void) {
    mxfa::unload_code_objects();
    return MXFA_OK;
}

int mxfa_set_code_object(const char *path) {
    mxfa::set_code_object_path(path);
    return MXFA_OK;
}

int mxfa_check_code_object(const char *path) {
    return mxfa::check_code_object(path) == mxfa::CodeObjectStatus::kOk ? MXFA_OK : MXFA_ERR_CODE_OBJECT;
}

int mxfa_check_shape(const mxfa_shape *shape) { return check_shape(shape); }

int mxfa_run_flash(const mxfa_shape *shape, const void *q, const void *k, const void *v, void *o,
                   void *stream) {
    return fwd_impl(shape, q, k, v, o, nullptr, false, stream);
}

int mxfa_run_flash_lse(const mxfa_shape *shape, const void *q, const void *k, const void *v, void *o,
                       float *lse, void *stream) {
    return fwd_impl(shape, q, k, v, o, lse, true, stream);
}

int mxfa_run_preprocess(const mxfa_shape *shape, const void *dout, const void *o, float *delta, void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({dout, o, delta});
    if (rc != MXFA_OK) return rc;
    Params p = make_params(shape);
    p.dout = dout;
    p.o_in = o;
    p.delta = delta;
    return from_hip(mxfa::launch_preprocess(p, shape->dtype == MXFA_BF16, shape->d,
                                            static_cast<hipStream_t>(stream)));
}

int mxfa_run_bwd_dq(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *dout,
                    const float *lse, const float *delta, void *dq, void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, k, v, dout, lse, delta, dq});
    if (rc != MXFA_OK) return rc;
    Params p = bwd_params(shape, q, k, v, dout, lse, delta);
    p.dq = dq;
    return from_hip(mxfa::launch_bwd_dq(p, shape->dtype == MXFA_BF16, shape->d, shape->causal, 0,
                                        static_cast<hipStream_t>(stream)));
}

int mxfa_run_bwd_dkv(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *dout,
                     const float *lse, const float *delta, void *dk, void *dv, void *stream) {
    return mxfa_run_bwd_dkv_ws(shape, q, k, v, dout, lse, delta, dk, dv, nullptr, 0, stream);
}

int mxfa_run_bwd_dkv_ws(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *dout,
                        const float *lse, const float *delta, void *dk, void *dv, void *workspace,
                        size_t workspace_bytes, void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, k, v, dout, lse, delta, dk, dv});
    if (rc != MXFA_OK) return rc;
    rc = check_workspace(shape, workspace, workspace_bytes);
    if (rc != MXFA_OK) return rc;
    Params p = bwd_params(shape, q, k, v, dout, lse, delta);
    p.dk = dk;
    p.dv = dv;
    p.dkv_ws = static_cast<float *>(workspace);
    return from_hip(mxfa::launch_bwd_dkv(p, shape->dtype == MXFA_BF16, shape->d, shape->causal,
                                         static_cast<hipStream_t>(stream)));
}

int mxfa_run_bwd_flash(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                       const void *dout, const float *lse, const float *delta, void *dq, void *dk, void *dv,
                       void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, k, v, dout, lse, delta, dq, dk, dv});
    if (rc != MXFA_OK) return rc;
    rc = mxfa_run_bwd_dkv(shape, q, k, v, dout, lse, delta, dk, dv, stream);
    if (rc != MXFA_OK) return rc;
    return mxfa_run_bwd_dq(shape, q, k, v, dout, lse, delta, dq, stream);
}

int mxfa_run_bwd_dq_delta(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                          const void *dout, const float *lse, float *delta, void *dq, void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, k, v, o, dout, lse, delta, dq});
    if (rc != MXFA_OK) return rc;
    Params p = bwd_params(shape, q, k, v, dout, lse, delta);
    p.o_in = o;
    p.dq = dq;
    return from_hip(mxfa::launch_bwd_dq(p, shape->dtype == MXFA_BF16, shape->d, shape->causal, 1,
                                        static_cast<hipStream_t>(stream)));
}

int mxfa_run_bwd(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                 const void *dout, const float *lse, float *delta, void *dq, void *dk, void *dv, void *stream) {
    return mxfa_run_bwd_ws(shape, q, k, v, o, dout, lse, delta, dq, dk, dv, nullptr, 0, stream);
}

int mxfa_run_bwd_ws(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, float *delta, void *dq, void *dk, void *dv,
                    void *workspace, size_t workspace_bytes, void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, k, v, o, dout, lse, delta, dq, dk, dv});
    if (rc != MXFA_OK) return rc;
    rc = check_workspace(shape, workspace, workspace_bytes);
    if (rc != MXFA_OK) return rc;
    {
        // the dQ and dK/dV work in one launch (plus the reduce of a GQA split)
        Params p = bwd_params(shape, q, k, v, dout, lse, delta);
        if (mxfa::bwd_fused_available(p, shape->dtype == MXFA_BF16, shape->d, static_cast<hipStream_t>(stream))) {
            p.o_in = o;
            p.dq = dq;
            p.dk = dk;
            p.dv = dv;
            p.dkv_ws = static_cast<float *>(workspace);
            return from_hip(mxfa::launch_bwd_fused(p, shape->d, shape->causal, static_cast<hipStream_t>(stream)));
        }
    }
    // dQ pass first: it computes Delta and writes it for the dK/dV pass
    rc = mxfa_run_bwd_dq_delta(shape, q, k, v, o, dout, lse, delta, dq, stream);
    if (rc != MXFA_OK) return rc;
    return mxfa_run_bwd_dkv_ws(shape, q, k, v, dout, lse, delta, dk, dv, workspace, workspace_bytes, stream);
}

size_t mxfa_bwd_noalloc_scratch_bytes(void) { return mxfa::noalloc_scratch_bytes(); }

int mxfa_run_bwd_noalloc(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                         const void *dout, const float *lse, float *delta, void *dq, void *dk, void *dv,
                         void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, k, v, o, dout, lse, delta, dq, dk, dv});
    if (rc != MXFA_OK) return rc;
    const size_t need = mxfa_bwd_workspace_bytes(shape);
    if (need > mxfa::noalloc_scratch_bytes()) return MXFA_ERR_SCRATCH;
    void *scratch = nullptr;
    if (need > 0) {
        int device = -1;
        if (hipGetDevice(&device) != hipSuccess) return MXFA_ERR_DEVICE;
        if (mxfa::noalloc_scratch(device, &scratch) != hipSuccess) return MXFA_ERR_DEVICE;
    }
    return mxfa_run_bwd_ws(shape, q, k, v, o, dout, lse, delta, dq, dk, dv, scratch, need, stream);
}

int mxfa_bwd_one_launch(const mxfa_shape *shape) {
    if (check_shape(shape) != MXFA_OK) return 0;
    const Params p = make_params(shape);
    return mxfa::bwd_fused_available(p, shape->dtype == MXFA_BF16, shape->d, nullptr) ? 1 : 0;
}

int mxfa_set_bwd_options(const mxfa_bwd_options *options) {
    if (options == nullptr) return MXFA_ERR_NULL;
    if (options->one_launch != 0 && options->one_launch != 1) return MXFA_ERR_SHAPE;
    if (options->reduce_wait_us < 0) return MXFA_ERR_SHAPE;
    mxfa::set_bwd_options(options->one_launch, options->delta_wait_us, options->reduce_wait_us);
    return MXFA_OK;
}

int mxfa_get_bwd_options(mxfa_bwd_options *options) {
    if (options == nullptr) return MXFA_ERR_NULL;
    mxfa::get_bwd_options(&options->one_launch, &options->delta_wait_us, &options->reduce_wait_us);
    return MXFA_OK;
}

int mxfa_bwd_delta_fallbacks(unsigned long long *count) {
    if (count == nullptr) return MXFA_ERR_NULL;
    const hipError_t e = mxfa::read_delta_fallbacks(count);
    if (e == hipSuccess) return MXFA_OK;
    return e == hipErrorInvalidImage ? MXFA_ERR_CODE_OBJECT : MXFA_ERR_DEVICE;
}

int mxfa_bwd_reduce_timeouts(unsigned long long *count) {
    if (count == nullptr) return MXFA_ERR_NULL;
    const hipError_t e = mxfa::read_reduce_timeouts(count);
    if (e == hipSuccess) return MXFA_OK;
    return e == hipErrorInvalidImage ? MXFA_ERR_CODE_OBJECT : MXFA_ERR_DEVICE;
}

size_t mxfa_bwd_workspace_bytes(const mxfa_shape *shape) {
    if (check_shape(shape) != MXFA_OK) return 0;
    const Params p = make_params(shape);
    // fp32 partial dK and dV planes, one pair per share of a key block, and a
    // flag per share
    return mxfa::dkv_workspace_bytes(p, shape->dtype == MXFA_BF16, shape->d, shape->causal);
}

int mxfa_run_bwd_naive(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                       const void *dout, const float *lse, const float *delta, void *dq, void *dk, void *dv,
                       void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    if (shape->dtype != MXFA_F32) return MXFA_ERR_UNSUPPORTED;
    rc = check_ptrs({q, k, v, dout, lse, delta, dq, dk, dv});
    if (rc != MXFA_OK) return rc;
    if ((long long)shape->B * shape->Hq > kMaxGridY) return MXFA_ERR_SHAPE;
    Params p = bwd_params(shape, q, k, v, dout, lse, delta);
    p.dq = dq;
    p.dk = dk;
    p.dv = dv;
    return from_hip(mxfa::launch_bwd_naive(p, shape->d, shape->causal, static_cast<hipStream_t>(stream)));
}

size_t mxfa_naive_scratch_bytes(const mxfa_shape *shape) {
    if (check_shape(shape) != MXFA_OK) return 0;
    return (size_t)shape->B * shape->Hq * (size_t)shape->N * (size_t)shape->N * sizeof(float);
}

int mxfa_run_naive_fwd(const mxfa_shape *shape, const void *q, const void *k, const void *v, float *s, void *o,
                       void *stream) {
    int rc = check_shape(shape);
    if (rc != MXFA_OK) return rc;
    if (shape->dtype != MXFA_F32) return MXFA_ERR_UNSUPPORTED;
    rc = check_ptrs({q, k, v, s, o});
    if (rc != MXFA_OK) return rc;
    if ((long long)shape->B * shape->Hq > kMaxGridY) return MXFA_ERR_SHAPE;
    if (((long long)shape->N + 15) / 16 > kMaxGridY) return MXFA_ERR_SHAPE;
    Params p = make_params(shape);
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    return from_hip(mxfa::launch_naive_fwd(p, s, shape->d, shape->causal, static_cast<hipStream_t>(stream)));
}

int mxfa_check_prefill(const mxfa_prefill_shape *s) {
    if (s == nullptr) return MXFA_ERR_NULL;
    if (s->dtype != MXFA_F32 && s->dtype != MXFA_BF16) return MXFA_ERR_DTYPE;
    if (s->n_tok < 1 || s->n_head < 1 || s->n_kv_head < 1 || s->head_dim < 1 || s->pos0 < 0) return MXFA_ERR_SHAPE;
    if (s->n_head % s->n_kv_head != 0) return MXFA_ERR_SHAPE;
    if (!(s->scale >= 0.0f) || std::isinf(s->scale)) return MXFA_ERR_SHAPE;
    // query positions (pos0 + row, the rows of a single-row call being its
    // GQA group's heads) stay inside int with a block to spare
    if ((long long)s->pos0 + std::max(s->n_tok, s->n_head) > 0x7fffffffLL - 128) return MXFA_ERR_SHAPE;
    // grid.y is the query blocks, 64 rows each in the smallest form a prefill
    // launches (fp32, paged d = 128, the split kernels); a single row's
    // blocks hold its GQA group's heads
    const long long rows = s->n_tok == 1 ? std::max(1, s->n_head / s->n_kv_head) : s->n_tok;
    if ((rows + 63) / 64 > kMaxGridY) return MXFA_ERR_SHAPE;
    if (s->head_dim != 64 && s->head_dim != 128) return MXFA_ERR_UNSUPPORTED;
    if (s->dtype == MXFA_F32 && s->head_dim != 64) return MXFA_ERR_UNSUPPORTED;
    // every head of a row must fit inside the row
    const long long qw = (long long)s->n_head * s->head_dim, kw = (long long)s->n_kv_head * s->head_dim;
    if (s->q_stride < qw || s->out_stride < qw || s->kv_stride < kw) return MXFA_ERR_SHAPE;
    // rows start on 16-byte boundaries (the kernels load and stage 16-byte chunks)
    const int esz = s->dtype == MXFA_BF16 ? 2 : 4;
    if (((long long)s->q_stride * esz) % 16 || ((long long)s->kv_stride * esz) % 16 ||
        ((long long)s->out_stride * esz) % 16)
        return MXFA_ERR_ALIGN;
    return MXFA_OK;
}

namespace {
// The forward's parameters for a prefill shape (checked by the caller).
Params prefill_params(const mxfa_prefill_shape *s, const void *q, const void *kcache, const void *vcache,
                      void *out) {
    mxfa_shape sh{1, s->n_head, s->n_kv_head, s->n_tok, s->head_dim, 1, s->dtype, s->scale};
    Params p = make_params(&sh);
    p.q = q;
    p.k = kcache;
    p.v = vcache;
    p.o = out;
    p.lse = nullptr;
    // token-major rows: head h at column h * head_dim of every row
    p.q_rs = s->q_stride;
    p.kv_rs = s->kv_stride;
    p.o_rs = s->out_stride;
    p.q_hs = p.o_hs = p.kv_hs = s->head_dim;
    p.q_bs = p.o_bs = p.kv_bs = 0;
    p.Nk = s->pos0 + s->n_tok;
    p.pos0 = s->pos0;
    p.prefill = 1;
    if (s->n_tok == 1 && s->n_head > s->n_kv_head) {
        // A single row (decode-like): the query heads of a GQA group become the
        // rows of one block per KV head, so each K/V stage staged serves the
        // whole group instead of one head. Row i sits at column (kvh group + i)
        // head_dim of the one Q / O row. With Nk = pos0 + 1 every row's causal
        // limit min(pos0 + i, Nk - 1) is pos0, as the row's own.
        const int group = s->n_head / s->n_kv_head;
        p.Hq = s->n_kv_head;
        p.group = 1;
        p.N = group;
        p.q_rs = p.o_rs = s->head_dim;
        p.q_hs = p.o_hs = (long long)group * s->head_dim;
    }
    return p;
}
}  // namespace

int mxfa_run_prefill(const mxfa_prefill_shape *s, const void *q, const void *kcache, const void *vcache, void *out,
                     void *stream) {
    int rc = mxfa_check_prefill(s);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, kcache, vcache, out});
    if (rc != MXFA_OK) return rc;
    const Params p = prefill_params(s, q, kcache, vcache, out);
    return from_hip(mxfa::launch_fwd(p, s->dtype == MXFA_BF16, s->head_dim, 1, static_cast<hipStream_t>(stream)));
}

namespace {
// The checks and parameters of a paged prefill (MXFA_OK and *p set, or the status).
int paged_params(const mxfa_prefill_shape *s, const void *q, const void *kcache, const void *vcache, void *out,
                 const int *block_table, int block_size, Params *p) {
    int rc = mxfa_check_prefill(s);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, kcache, vcache, out});
    if (rc != MXFA_OK) return rc;
    if (block_table == nullptr) return MXFA_ERR_NULL;
    if (reinterpret_cast<uintptr_t>(block_table) % alignof(int) != 0) return MXFA_ERR_ALIGN;
    // block sizes are powers of two (the reference engine's is 16)
    if (block_size < 1 || block_size > (1 << 24) || (block_size & (block_size - 1)) != 0) return MXFA_ERR_UNSUPPORTED;
    *p = prefill_params(s, q, kcache, vcache, out);
    p->block_table = block_table;
    while ((1 << p->bs_shift) < block_size) ++p->bs_shift;
    return MXFA_OK;
}

// The split launch when the shape gains from one, else the unsplit one
// (p.block_table, if set, selects the paged kernels).
int run_prefill_maybe_split(const mxfa_prefill_shape *s, Params p, void *workspace, size_t workspace_bytes,
                            void *stream) {
    const int dtype_bf16 = s->dtype == MXFA_BF16;
    const int splits = mxfa::fwd_splits(p, dtype_bf16, s->head_dim);
    if (splits <= 1)  // the unsplit launch: no workspace needed or read
        return from_hip(mxfa::launch_fwd(p, dtype_bf16, s->head_dim, 1, static_cast<hipStream_t>(stream)));
    if (workspace == nullptr) return MXFA_ERR_NULL;
    if (!aligned16(workspace)) return MXFA_ERR_ALIGN;
    if (workspace_bytes < mxfa::fwd_split_workspace_bytes(p, s->head_dim, splits)) return MXFA_ERR_WORKSPACE;
    p.fwd_part = static_cast<float *>(workspace);
    return from_hip(mxfa::launch_fwd_split(p, dtype_bf16, s->head_dim, splits, static_cast<hipStream_t>(stream)));
}
}  // namespace

size_t mxfa_prefill_workspace_bytes(const mxfa_prefill_shape *s) {
    if (mxfa_check_prefill(s) != MXFA_OK) return 0;
    const Params p = prefill_params(s, nullptr, nullptr, nullptr, nullptr);
    const int dtype_bf16 = s->dtype == MXFA_BF16;
    return mxfa::fwd_split_workspace_bytes(p, s->head_dim, mxfa::fwd_splits(p, dtype_bf16, s->head_dim));
}

int mxfa_run_prefill_ws(const mxfa_prefill_shape *s, const void *q, const void *kcache, const void *vcache, void *out,
                        void *workspace, size_t workspace_bytes, void *stream) {
    int rc = mxfa_check_prefill(s);
    if (rc != MXFA_OK) return rc;
    rc = check_ptrs({q, kcache, vcache, out});
    if (rc != MXFA_OK) return rc;
    return run_prefill_maybe_split(s, prefill_params(s, q, kcache, vcache, out), workspace, workspace_bytes, stream);
}

int mxfa_run_prefill_paged(const mxfa_prefill_shape *s, const void *q, const void *kcache, const void *vcache,
                           void *out, const int *block_table, int block_size, void *stream) {
    Params p;
    const int rc = paged_params(s, q, kcache, vcache, out, block_table, block_size, &p);
    if (rc != MXFA_OK) return rc;
    return from_hip(mxfa::launch_fwd(p, s->dtype == MXFA_BF16, s->head_dim, 1, static_cast<hipStream_t>(stream)));
}

int mxfa_run_prefill_paged_ws(const mxfa_prefill_shape *s, const void *q, const void *kcache, const void *vcache,
                              void *out, const int *block_table, int block_size, void *workspace,
                              size_t workspace_bytes, void *stream) {
    Params p;
    const int rc = paged_params(s, q, kcache, vcache, out, block_table, block_size, &p);
    if (rc != MXFA_OK) return rc;
    return run_prefill_maybe_split(s, p, workspace, workspace_bytes, stream);
}

int mxfa_probe_sink_len(void) { return mxfa::probe_sink_len(); }

int mxfa_probe_mfma(int dtype, int iters, float *sink, double *flops, void *stream) {
    if (dtype != MXFA_F32 && dtype != MXFA_BF16) return MXFA_ERR_DTYPE;
    if (iters < 1) return MXFA_ERR_SHAPE;
    if (sink == nullptr || flops == nullptr) return MXFA_ERR_NULL;
    if (!aligned16(sink)) return MXFA_ERR_ALIGN;
    *flops = mxfa::probe_mfma_flops(dtype == MXFA_BF16, iters);
    return from_hip(mxfa::launch_probe_mfma(dtype == MXFA_BF16, iters, sink, static_cast<hipStream_t>(stream)));
}

int mxfa_probe_mfma32(int iters, float *sink, double *flops, void *stream) {
    if (iters < 1) return MXFA_ERR_SHAPE;
    if (sink == nullptr || flops == nullptr) return MXFA_ERR_NULL;
    if (!aligned16(sink)) return MXFA_ERR_ALIGN;
    *flops = mxfa::probe_mfma32_flops(iters);
    return from_hip(mxfa::launch_probe_mfma32(iters, sink, static_cast<hipStream_t>(stream)));
}

int mxfa_probe_mix(int mix, int waves_per_simd, int iters, float *sink, double *flops, void *stream) {
    if (mix < 0 || mix >= mxfa::probe_mix_count() || waves_per_simd < 1 || waves_per_simd > 8 || iters < 1)
        return MXFA_ERR_SHAPE;
    if (sink == nullptr || flops == nullptr) return MXFA_ERR_NULL;
    if (!aligned16(sink)) return MXFA_ERR_ALIGN;
    *flops = mxfa::probe_mix_flops(waves_per_simd, iters);
    return from_hip(mxfa::launch_probe_mix(mix, waves_per_simd, iters, sink, static_cast<hipStream_t>(stream)));
}

int mxfa_probe_wg_times(void *dst, size_t bytes, size_t *avail) {
    if (avail == nullptr) return MXFA_ERR_NULL;
    const hipError_t e = mxfa::read_wg_times(dst, bytes, avail);
    if (e == hipErrorNotFound) return MXFA_ERR_UNSUPPORTED;
    return from_hip(e);
}

int mxfa_probe_read(const void *x, size_t bytes, float *sink, void *stream) {
    int rc = check_ptrs({x, sink});
    if (rc != MXFA_OK) return rc;
    if (bytes == 0 || bytes % 16 != 0) return MXFA_ERR_SHAPE;
    return from_hip(mxfa::launch_probe_read(x, bytes, sink, static_cast<hipStream_t>(stream)));
}

int mxfa_probe_copy(const void *x, void *y, size_t bytes, void *stream) {
    int rc = check_ptrs({x, y});
    if (rc != MXFA_OK) return rc;
    if (bytes == 0 || bytes % 16 != 0) return MXFA_ERR_SHAPE;
    return from_hip(mxfa::launch_probe_copy(x, y, bytes, static_cast<hipStream_t>(stream)));
}

int mxfa_probe_dq_atomic(float *acc, int bh, int n, int atomic, double *bytes, void *stream) {
    int rc = check_ptrs({acc, bytes});
    if (rc != MXFA_OK) return rc;
    if (bh < 1 || n < 128 || n % 128 != 0 || n / 128 > kMaxGridY) return MXFA_ERR_SHAPE;
    if (atomic != 0 && atomic != 1) return MXFA_ERR_SHAPE;
    *bytes = mxfa::probe_dq_atomic_bytes(bh, n);
    return from_hip(mxfa::launch_probe_dq_atomic(acc, bh, n, atomic, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
