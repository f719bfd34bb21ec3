// Dense FP8 block-quantized GEMM (placeholder translation unit; kernels follow).
#include "common.h"
