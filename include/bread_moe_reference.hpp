/* bread_moe_reference.hpp - the reference's own C++ declaration of
 * bread_matvec, defined by libbread_moe.so, so that a HIP build of the
 * reference's translation units links against this library without editing
 * their declarations or call sites.
 *
 * one_layer.cu:46-47, main.cu:65-66 and expert_bench.cu:15-16 declare
 *
 *     extern void bread_matvec(void *w, half *x, half *y,
 *                              int rows, int cols, int qtype, cudaStream_t stream);
 *
 * with C++ linkage (kernels.cu:289 defines it).  In a HIP build `half` is
 * __half and `cudaStream_t` is hipStream_t; the library defines exactly that
 * overload, beside the extern "C" bread_matvec of bread_moe.h (whose
 * parameter types differ: const weights, uint16_t activations, an int
 * status).  The overload keeps the reference's error behaviour: an unknown
 * qtype or a failed launch prints the reason and calls exit(1)
 * (kernels.cu:303-307).  A caller need not include this header; its own
 * declaration resolves to the same symbol.
 */
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include "bread_moe.h"

void bread_matvec(void *w, __half *x, __half *y, int rows, int cols, int qtype, hipStream_t stream);
