/* Challenge adapters: one shared library per challenge, each exporting a C
 * function named `solve` (plus opw_solve_last_error). Pointers are device
 * pointers; every solve synchronizes the device before it returns. A contract
 * violation leaves outputs untouched, prints one line to stderr and is kept
 * in opw_solve_last_error() ("" after a successful call).
 *
 * Because all six share the symbol name, their signatures are given below as
 * function-pointer types; bind them with dlopen/ctypes per library:
 *
 *   libopw_solve_vector_add.so           opw_solve_vector_add_fn
 *       replaces tests/integration/vector_add.cu:7
 *   libopw_solve_relu.so                 opw_solve_relu_fn
 *       replaces tests/integration/relu.cu:7
 *   libopw_solve_reduction.so            opw_solve_reduction_fn
 *       replaces tests/integration/reduction.cu:10
 *   libopw_solve_softmax.so              opw_solve_softmax_fn
 *       replaces tests/integration/softmax.cu:3
 *   libopw_solve_layer_normalization.so  opw_solve_layer_normalization_fn
 *       replaces tests/integration/layer_normalization.cu:3-4
 *   libopw_solve_matrix_multiplication.so opw_solve_matrix_multiplication_fn
 *       replaces tests/integration/matrix_multiplication.cu:3
 */
#ifndef OPWORKS_SOLVE_H
#define OPWORKS_SOLVE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void (*opw_solve_vector_add_fn)(const float *a, const float *b, float *out, size_t n);
typedef void (*opw_solve_relu_fn)(const float *in, float *out, int n);
typedef void (*opw_solve_reduction_fn)(const float *in, float *out, int n);
typedef void (*opw_solve_softmax_fn)(const float *in, float *out, int n);
typedef void (*opw_solve_layer_normalization_fn)(const float *in, const float *gamma, const float *beta, float *out,
                                                 int rows, int cols, float eps);
typedef void (*opw_solve_matrix_multiplication_fn)(const float *a, const float *b, float *out, int m, int n, int k);

/* Exported by every adapter library: message of the calling thread's last
 * failed solve in that library. */
const char *opw_solve_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
