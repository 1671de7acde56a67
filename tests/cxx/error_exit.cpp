// Calls one include/kernels.h entry point with arguments the library rejects
// on the host (before any GPU call), to check the reference's error
// convention (FINAL_CLEAN_CODE/include/common.h:20-30): the call prints
// "HIP error at <file>:<line> — <message>" to stderr and exits with
// EXIT_FAILURE.  Run by tests/test_cxx_error_exit.py; needs no GPU.
#include <cstdio>
#include <cstring>

#include "kernels.h"

int main(int argc, char** argv) {
    const char* which = argc > 1 ? argv[1] : "";
    if (!std::strcmp(which, "layernorm_forward"))
        layernorm_forward(nullptr, nullptr, nullptr, nullptr, -1, 768);
    else if (!std::strcmp(which, "layernorm_backward"))
        layernorm_backward(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                           8, -3);
    else if (!std::strcmp(which, "bias_gelu_forward"))
        bias_gelu_forward(nullptr, nullptr, nullptr, 4, 0);
    else if (!std::strcmp(which, "residual_add"))
        residual_add(nullptr, nullptr, nullptr, -5);
    else if (!std::strcmp(which, "embedding_backward"))
        embedding_backward(nullptr, nullptr, nullptr, 16, 0);
    else if (!std::strcmp(which, "layernorm_forward_save_null"))
        layernorm_forward_save(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 4, 8);
    else {
        std::fprintf(stderr, "unknown case %s\n", which);
        return 2;
    }
    std::printf("returned normally\n");  // not reached: the call exits
    return 0;
}
