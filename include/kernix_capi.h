/* kernix_capi.h — the ctypes-facing C ABI of libkernix.so (MI355X build).
 *
 * The first ten entry points are the reference's exports with identical signatures, argument meaning and return
 * values; each line cites the reference definition it replaces (reference src/kernix_capi.c).  The Python binding
 * binds them exactly as the reference binding does (reference python/kernix.py:21-40).
 */
#ifndef KERNIX_CAPI_H
#define KERNIX_CAPI_H

#include <stddef.h>

#include "kernix_model.h"

#ifdef __cplusplus
extern "C" {
#endif

KERNIX_API kernix_model* kernix_capi_load(const char* path);                        /* src/kernix_capi.c:7 */
KERNIX_API void kernix_capi_free(kernix_model* m);                                  /* src/kernix_capi.c:9 */
KERNIX_API void kernix_capi_trim(kernix_model* m);                                  /* src/kernix_capi.c:12 */
KERNIX_API void kernix_capi_set_workspace_limit(kernix_model* m, size_t bytes);     /* src/kernix_capi.c:15 */
KERNIX_API void kernix_capi_dims(const kernix_model* m, int* in_dim, int* out_dim, int* seq_len); /* :17-20 */
KERNIX_API int kernix_capi_forward(kernix_model* m, const float* x, int rows, float* out);          /* :24-32 */
KERNIX_API int kernix_capi_set_ane(kernix_model* m, int on);                        /* src/kernix_capi.c:35 (-1) */
KERNIX_API void kernix_capi_ane_info(const kernix_model* m, int* out4);             /* src/kernix_capi.c:38-43 */
KERNIX_API int kernix_capi_ane_dump(const kernix_model* m, int seg, int batch, const char* path); /* :46-54 (-1) */
KERNIX_API void kernix_capi_shapes(const kernix_model* m, int* in_nd, int* in_shape4, int* out_nd, int* out_shape4,
                                   int* layout);                                    /* src/kernix_capi.c:57-61 */

/* Extensions (no counterpart in the reference ABI). */
KERNIX_API int kernix_capi_set_int8_mode(kernix_model* m, int mode);  /* KERNIX_INT8_REF / KERNIX_INT8_I8; 0 or -1 */
/* Forward on device buffers (rows × in_dim → (rows/seq_len) × out_dim), stream = hipStream_t or NULL; enqueues only. */
KERNIX_API int kernix_capi_forward_device(kernix_model* m, const float* d_x, int rows, float* d_out, void* stream);
/* kernix_capi_forward with each sample of x channels-first (kernix_model_forward_cf): the transpose runs on the GPU. */
KERNIX_API int kernix_capi_forward_cf(kernix_model* m, const float* x, int rows, float* out);
/* Waits for the last forward; -1 if a device forward since the previous call must be run again (kernix_model.h). */
KERNIX_API int kernix_capi_device_status(kernix_model* m);
/* Workspace accounting: floats per sample, batch-independent floats, rows of the current workspace (-1 = none). */
KERNIX_API void kernix_capi_ws_info(const kernix_model* m, size_t* per_sample, size_t* fixed, int* batch);

#ifdef __cplusplus
}
#endif

#endif
