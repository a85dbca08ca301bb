// Stage kernels (pipe_gemm*, pipe_layer_norm, pipe_add, pipe_concat).
#include "gp_host.hpp"
