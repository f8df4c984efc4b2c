// vo_memory.cpp -- the memory ops of the Backend trait: the activation
// workspace (alloc_workspace / workspace_elems, crates/engine/src/backend/
// mod.rs:76-78), device-resident weights (upload / weight_shape, mod.rs:69-72)
// and the debug read of a workspace region (read, mod.rs:177-181).
//
// With these an engine that links only this library gets all of its device
// memory from it: the workspace its arena carves into Regions, the weights,
// the KV pool (vo_kv_pool_create) and the step metadata (vo_step_meta_create).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "vo_backend.hpp"

using namespace vo;

struct vo_workspace {
    int device = 0;
    uint64_t elems = 0;
    uint8_t *base = nullptr;  // elems * kWorkspaceElemBytes bytes
};

struct vo_weight {
    int device = 0;
    int32_t dtype = VO_DTYPE_BF16;
    std::vector<uint64_t> shape;
    uint64_t numel = 0;
    void *data = nullptr;
};

namespace {

constexpr uint64_t kWorkspaceElemBytes = 4;  // one f32 element of the reference's workspace

uint64_t dtype_bytes(int32_t dtype) { return dtype == VO_DTYPE_F32 ? 4 : 2; }

// f32 -> bf16 bits, round to nearest even; NaN stays a (quiet) NaN.
uint16_t f32_to_bf16_host(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if (std::isnan(f)) return static_cast<uint16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

float bf16_to_f32_host(uint16_t b) {
    const uint32_t u = static_cast<uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// cpu/mod.rs:57-62 (check_in_workspace): offset + rows * cols elements must
// lie inside the workspace, whatever the element type the op reads there.
vo_status check_region(const vo_workspace *ws, const char *op, uint64_t offset, uint64_t rows,
                       uint64_t cols) {
    const uint64_t len = rows * cols;
    if ((cols && len / cols != rows) || offset > ws->elems || len > ws->elems - offset) {
        Error e;
        e.status = VO_ERR_OUTSIDE_WORKSPACE;
        e.op = op;
        e.value = offset;
        e.limit = ws->elems;
        e.message = "region outside the workspace (workspace not allocated, or too small)";  // error.rs:47
        return fail(e);
    }
    return VO_OK;
}

vo_status check_dtype(const char *op, int32_t dtype) {
    if (dtype != VO_DTYPE_BF16 && dtype != VO_DTYPE_F32)
        return fail_argument(op, "dtype must be VO_DTYPE_BF16 or VO_DTYPE_F32");
    return VO_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Workspace
// ---------------------------------------------------------------------------

extern "C" int32_t vo_workspace_create(int32_t device, uint64_t elems, vo_workspace **out) {
    const char *op = "alloc_workspace";
    if (!out) return fail_argument(op, "null output");
    *out = nullptr;
    if (elems > (~0ull) / kWorkspaceElemBytes) return fail_capacity("workspace elements", elems, (~0ull) / kWorkspaceElemBytes);
    DeviceGuard guard(device);
    if (!guard.ok()) return fail_device(op, hipErrorInvalidDevice, "hipSetDevice");
    vo_workspace *ws = new (std::nothrow) vo_workspace();
    if (!ws) return fail_argument(op, "out of host memory");
    ws->device = device;
    ws->elems = elems;
    if (elems) {
        const uint64_t bytes = elems * kWorkspaceElemBytes;
        hipError_t err = hipMalloc(reinterpret_cast<void **>(&ws->base), bytes);
        // Zero-filled, as the reference's (cpu/mod.rs:163-166).
        if (err == hipSuccess) err = hipMemset(ws->base, 0, bytes);
        if (err != hipSuccess) {
            if (ws->base) (void)hipFree(ws->base);
            delete ws;
            return fail_device(op, err, hipGetErrorString(err));
        }
    }
    *out = ws;
    clear_error();
    return VO_OK;
}

extern "C" void vo_workspace_destroy(vo_workspace *ws) {
    if (!ws) return;
    DeviceGuard guard(ws->device);
    if (ws->base) (void)hipFree(ws->base);
    delete ws;
}

extern "C" uint64_t vo_workspace_elems(const vo_workspace *ws) { return ws ? ws->elems : 0; }

extern "C" int32_t vo_workspace_region(const vo_workspace *ws, uint64_t offset, uint64_t rows,
                                       uint64_t cols, void **ptr) {
    const char *op = "region";
    if (!ws || !ptr) return fail_argument(op, "null workspace or output");
    *ptr = nullptr;
    if (vo_status rc = check_region(ws, op, offset, rows, cols)) return rc;
    *ptr = ws->base + offset * kWorkspaceElemBytes;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_workspace_read(const vo_workspace *ws, uint64_t offset, uint64_t rows,
                                     uint64_t cols, int32_t dtype, float *host_out, void *stream) {
    const char *op = "read";
    if (!ws) return fail_argument(op, "null workspace");
    if (vo_status rc = check_dtype(op, dtype)) return rc;
    if (vo_status rc = check_region(ws, op, offset, rows, cols)) return rc;
    const uint64_t n = rows * cols;
    if (n == 0) {
        clear_error();
        return VO_OK;
    }
    if (!host_out) return fail_argument(op, "null host output");
    DeviceGuard guard(ws->device);
    // Debug and tests only (mod.rs:177-181): waits for the stream, then copies.
    hipError_t err = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    const uint8_t *src = ws->base + offset * kWorkspaceElemBytes;
    if (err == hipSuccess) {
        if (dtype == VO_DTYPE_F32) {
            err = hipMemcpy(host_out, src, n * 4, hipMemcpyDeviceToHost);
        } else {
            std::vector<uint16_t> tmp(n);
            err = hipMemcpy(tmp.data(), src, n * 2, hipMemcpyDeviceToHost);
            if (err == hipSuccess)
                for (uint64_t i = 0; i < n; ++i) host_out[i] = bf16_to_f32_host(tmp[i]);
        }
    }
    return device_status(op, err);
}

// ---------------------------------------------------------------------------
// Weights
// ---------------------------------------------------------------------------

extern "C" int32_t vo_weight_upload(int32_t device, const float *data, const uint64_t *shape,
                                    uint64_t ndim, int32_t dtype, vo_weight **out) {
    const char *op = "upload";
    if (!out) return fail_argument(op, "null output");
    *out = nullptr;
    if (vo_status rc = check_dtype(op, dtype)) return rc;
    if (ndim == 0 || !shape) return fail_shape(op, "a weight has at least one dimension");
    uint64_t numel = 1;
    for (uint64_t i = 0; i < ndim; ++i) {
        if (shape[i] && numel > (~0ull) / 4 / shape[i])
            return fail_capacity("weight elements", ~0ull, (~0ull) / 4);
        numel *= shape[i];
    }
    if (numel && !data) return fail_argument(op, "null data");
    DeviceGuard guard(device);
    if (!guard.ok()) return fail_device(op, hipErrorInvalidDevice, "hipSetDevice");
    vo_weight *w = new (std::nothrow) vo_weight();
    if (!w) return fail_argument(op, "out of host memory");
    w->device = device;
    w->dtype = dtype;
    w->shape.assign(shape, shape + ndim);
    w->numel = numel;
    hipError_t err = hipSuccess;
    if (numel) {
        const uint64_t bytes = numel * dtype_bytes(dtype);
        err = hipMalloc(&w->data, bytes);
        if (err == hipSuccess) {
            if (dtype == VO_DTYPE_F32) {
                err = hipMemcpy(w->data, data, bytes, hipMemcpyHostToDevice);
            } else {
                // Rounded on the host in slices, so the host copy stays small.
                constexpr uint64_t kSlice = 1ull << 22;
                std::vector<uint16_t> tmp(std::min<uint64_t>(numel, kSlice));
                for (uint64_t i0 = 0; i0 < numel && err == hipSuccess; i0 += kSlice) {
                    const uint64_t n = std::min<uint64_t>(kSlice, numel - i0);
                    for (uint64_t i = 0; i < n; ++i) tmp[i] = f32_to_bf16_host(data[i0 + i]);
                    err = hipMemcpy(static_cast<uint16_t *>(w->data) + i0, tmp.data(), n * 2,
                                    hipMemcpyHostToDevice);
                }
            }
        }
    }
    if (err != hipSuccess) {
        if (w->data) (void)hipFree(w->data);
        delete w;
        return fail_device(op, err, hipGetErrorString(err));
    }
    *out = w;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_weight_concat_rows(const vo_weight *const *parts, uint64_t count,
                                         vo_weight **out) {
    const char *op = "upload";
    if (!parts || !out || count == 0) return fail_argument(op, "null or empty parts");
    *out = nullptr;
    const vo_weight *p0 = parts[0];
    if (!p0) return fail_argument(op, "null part");
    uint64_t rows = 0;
    for (uint64_t i = 0; i < count; ++i) {
        const vo_weight *p = parts[i];
        if (!p) return fail_argument(op, "null part");
        if (p->shape.size() != 2 || p->dtype != p0->dtype || p->device != p0->device ||
            p->shape[1] != p0->shape[1])
            return fail_shape(op, "parts must be matrices of one dtype and device with the same "
                                  "number of columns");
        rows += p->shape[0];
    }
    DeviceGuard guard(p0->device);
    vo_weight *w = new (std::nothrow) vo_weight();
    if (!w) return fail_argument(op, "out of host memory");
    w->device = p0->device;
    w->dtype = p0->dtype;
    w->shape = {rows, p0->shape[1]};
    w->numel = rows * p0->shape[1];
    const uint64_t esz = dtype_bytes(w->dtype);
    hipError_t err = w->numel ? hipMalloc(&w->data, w->numel * esz) : hipSuccess;
    uint64_t at = 0;
    for (uint64_t i = 0; i < count && err == hipSuccess; ++i) {
        const uint64_t bytes = parts[i]->numel * esz;
        if (bytes)
            err = hipMemcpy(static_cast<uint8_t *>(w->data) + at, parts[i]->data, bytes,
                            hipMemcpyDeviceToDevice);
        at += bytes;
    }
    if (err != hipSuccess) {
        if (w->data) (void)hipFree(w->data);
        delete w;
        return fail_device(op, err, hipGetErrorString(err));
    }
    *out = w;
    clear_error();
    return VO_OK;
}

extern "C" void vo_weight_destroy(vo_weight *w) {
    if (!w) return;
    DeviceGuard guard(w->device);
    if (w->data) (void)hipFree(w->data);
    delete w;
}

extern "C" int32_t vo_weight_shape(const vo_weight *w, uint64_t *shape, uint64_t capacity,
                                   uint64_t *ndim) {
    if (!w || !ndim) return fail_argument("weight_shape", "null weight or ndim");
    *ndim = w->shape.size();
    if (shape)
        for (uint64_t i = 0; i < std::min<uint64_t>(capacity, w->shape.size()); ++i) shape[i] = w->shape[i];
    clear_error();
    return VO_OK;
}

extern "C" const void *vo_weight_data(const vo_weight *w) { return w ? w->data : nullptr; }

extern "C" int32_t vo_weight_dtype(const vo_weight *w) { return w ? w->dtype : -1; }
