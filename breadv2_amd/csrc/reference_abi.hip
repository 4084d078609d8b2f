// reference_abi.hip — the reference's C++ bread_matvec (kernels.cu:289,
// declared by one_layer.cu:46-47, main.cu:65-66, expert_bench.cu:15-16) on
// top of the C entry point, with the reference's print-and-exit on error
// (kernels.cu:303-307).  Declared in include/bread_moe_reference.hpp.
#include <stdio.h>
#include <stdlib.h>

#include "../../include/bread_moe_reference.hpp"

void bread_matvec(void *w, __half *x, __half *y, int rows, int cols, int qtype, hipStream_t stream)
{
    const int rc = bread_matvec(static_cast<const void *>(w), reinterpret_cast<const uint16_t *>(x),
                                reinterpret_cast<uint16_t *>(y), rows, cols, qtype, stream);
    if (rc != BREAD_OK) {
        fprintf(stderr, "bread_matvec: %s\n", bread_last_error());
        exit(1);
    }
}
