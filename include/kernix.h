/* kernix.h — portable tensor subset of the KERNIX C API, MI355X build.
 *
 * Keeps the reference's 2-D tensor structs and activation numbering (the numbering is part of the .knx file ABI):
 *   float_tensor / int_tensor / uint8_tensor   reference include/kernix.h:39-58
 *   kernix_float_new / float_zeros / float_free reference include/kernix.h:146-176, :209-227
 *   KERNIX_ACT_*                               reference include/kernix.h:928-942
 *
 * In this build a float_tensor either holds host memory (tensors created with kernix_float_new, model inputs and
 * outputs) or device memory (model workspace views, dequantized weight copies); the owner says which.  Host tensors are
 * 64-byte aligned so the HIP runtime can DMA from them without bouncing through an unaligned staging path.
 */
#ifndef KERNIX_H
#define KERNIX_H

#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KERNIX_API __attribute__((visibility("default")))

typedef struct {
    int row;
    int col;
    float* tensor;
} float_tensor;

typedef struct {
    int row;
    int col;
    int* tensor;
} int_tensor;

typedef struct {
    int row;
    int col;
    uint8_t* tensor;
} uint8_tensor;

/* Activation ids: identical to the .knx file format (KNX1/2 use 0-4, KNX3 all). */
enum {
    KERNIX_ACT_NONE = -1,
    KERNIX_ACT_RELU,
    KERNIX_ACT_GELU,         /* x/2·(1+erf(x/√2)), erf by Abramowitz–Stegun 7.1.26 */
    KERNIX_ACT_SILU,
    KERNIX_ACT_SIGMOID,
    KERNIX_ACT_TANH,
    KERNIX_ACT_LEAKY_RELU,   /* x < 0 ? alpha·x : x */
    KERNIX_ACT_ELU,          /* x < 0 ? alpha·(eˣ−1) : x */
    KERNIX_ACT_SELU,
    KERNIX_ACT_SOFTPLUS,
    KERNIX_ACT_RELU6,
    KERNIX_ACT_HARD_SIGMOID, /* relu6(x+3)/6 */
    KERNIX_ACT_HARD_SWISH,   /* x·relu6(x+3)/6 */
    KERNIX_ACT_GELU_TANH,
    KERNIX_ACT_EXP,
    KERNIX_ACT_MISH,
    KERNIX_ACT_SOFTSIGN,
    KERNIX_ACT_LAST = KERNIX_ACT_SOFTSIGN
};

/* Host tensor of rows×cols floats (zero-filled if zero != 0). NULL on failure or negative sizes. */
KERNIX_API float_tensor* kernix_float_new(int rows, int cols, int zero);
KERNIX_API float_tensor* float_zeros(int rows, int cols);
KERNIX_API void float_free(float_tensor* t);

#ifdef __cplusplus
}
#endif

#endif
