/* knx_capi.c — the ctypes-facing C ABI of libkernix.so: the reference's ten exports with identical signatures,
 * argument meaning and return values (reference src/kernix_capi.c:7-61).  The Python binding
 * (kernix_amd/kernix.py) and any C caller of the reference library bind these unchanged. */
#include <string.h>

#include "kernix_capi.h"
#include "knx_internal.h"

/* reference src/kernix_capi.c:7 */
KERNIX_API kernix_model* kernix_capi_load(const char* path) { return kernix_model_load(path); }

/* reference src/kernix_capi.c:9 */
KERNIX_API void kernix_capi_free(kernix_model* m) { kernix_model_free(m); }

/* reference src/kernix_capi.c:12: releases the device workspace, keeps the weights */
KERNIX_API void kernix_capi_trim(kernix_model* m) { kernix_model_trim(m); }

/* reference src/kernix_capi.c:15: bytes, 0 = unlimited; larger batches run in chunks */
KERNIX_API void kernix_capi_set_workspace_limit(kernix_model* m, size_t bytes) { kernix_model_set_workspace_limit(m, bytes); }

/* reference src/kernix_capi.c:17-20 */
KERNIX_API void kernix_capi_dims(const kernix_model* m, int* in_dim, int* out_dim, int* seq_len)
{
    *in_dim = m->in_dim;
    *out_dim = m->out_dim;
    *seq_len = m->seq_len;
}

/* reference src/kernix_capi.c:24-32: x is rows × in_dim (rows a positive multiple of seq_len); the
 * (rows/seq_len) × out_dim result is copied into the caller's out.  0 or -1. */
KERNIX_API int kernix_capi_forward(kernix_model* m, const float* x, int rows, float* out)
{
    if (m == NULL || x == NULL || out == NULL || rows <= 0) return -1;
    const float_tensor in = { rows, m->in_dim, (float*)x }; /* forward does not modify its input */
    const float_tensor* y = kernix_model_forward(m, &in);
    if (y == NULL) return -1;
    knx_copy_parallel(out, y->tensor, sizeof(float) * (size_t)y->row * (size_t)y->col);
    return 0;
}

/* kernix_capi_forward on channels-first samples (an extension: the axis moved on the device) */
KERNIX_API int kernix_capi_forward_cf(kernix_model* m, const float* x, int rows, float* out)
{
    if (m == NULL || x == NULL || out == NULL || rows <= 0) return -1;
    const float_tensor in = { rows, m->in_dim, (float*)x };
    const float_tensor* y = kernix_model_forward_cf(m, &in);
    if (y == NULL) return -1;
    knx_copy_parallel(out, y->tensor, sizeof(float) * (size_t)y->row * (size_t)y->col);
    return 0;
}

/* reference src/kernix_capi.c:35: the Neural Engine assist does not exist here: -1 ("unavailable") */
KERNIX_API int kernix_capi_set_ane(kernix_model* m, int on) { return kernix_model_set_ane(m, on); }

/* reference src/kernix_capi.c:38-43: segments, compiles, ane_runs, failures (all 0) */
KERNIX_API void kernix_capi_ane_info(const kernix_model* m, int* out)
{
    kernix_ane_info i;
    kernix_model_ane_info(m, &i);
    out[0] = i.segments;
    out[1] = i.compiles;
    out[2] = i.ane_runs;
    out[3] = i.failures;
}

/* reference src/kernix_capi.c:46-54: Core ML export is not available in this build: -1 */
KERNIX_API int kernix_capi_ane_dump(const kernix_model* m, int seg, int batch, const char* path)
{
    (void)m; (void)seg; (void)batch; (void)path;
    return -1;
}

/* reference src/kernix_capi.c:57-61 */
KERNIX_API void kernix_capi_shapes(const kernix_model* m, int* in_nd, int* in_shape, int* out_nd, int* out_shape, int* layout)
{
    *in_nd = m->in_nd;
    *out_nd = m->out_nd;
    *layout = m->layout;
    for (int k = 0; k < KERNIX_MAX_DIMS; k++) {
        in_shape[k] = m->in_shape[k];
        out_shape[k] = m->out_shape[k];
    }
}

/* Extensions (no counterpart in the reference ABI). */
KERNIX_API int kernix_capi_set_int8_mode(kernix_model* m, int mode) { return kernix_model_set_int8_mode(m, mode); }

/* d_x, d_out: device pointers; stream: hipStream_t or NULL (the model's stream). Enqueues and returns. */
KERNIX_API int kernix_capi_forward_device(kernix_model* m, const float* d_x, int rows, float* d_out, void* stream)
{
    return kernix_model_forward_device(m, d_x, rows, d_out, stream);
}

KERNIX_API int kernix_capi_device_status(kernix_model* m) { return kernix_model_device_status(m); }

/* Workspace accounting, for tests of the chunking rules: floats per sample, batch-independent floats, current batch. */
KERNIX_API void kernix_capi_ws_info(const kernix_model* m, size_t* per_sample, size_t* fixed, int* batch)
{
    *per_sample = m->ws_per_sample;
    *fixed = m->ws_fixed;
    *batch = m->batch;
}
