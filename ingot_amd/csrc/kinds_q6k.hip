// Per-format kernels (see kind_launch.h): GGML type 14 (Q6_K).
#include "kind_launch.cuh"

INGOT_INSTANTIATE_KIND(14)
INGOT_INSTANTIATE_F16(14)
