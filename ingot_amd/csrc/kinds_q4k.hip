// Per-format kernels (see kind_launch.h): GGML type 12 (Q4_K).
#include "kind_launch.cuh"

INGOT_INSTANTIATE_KIND(12)
INGOT_INSTANTIATE_FUSED(12, 12)
INGOT_INSTANTIATE_F16(12)
