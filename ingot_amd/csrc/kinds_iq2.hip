// Per-format kernels (see kind_launch.h): GGML types 16 17 22.
#include "kind_launch.cuh"

INGOT_INSTANTIATE_KIND(16)
INGOT_INSTANTIATE_KIND(17)
INGOT_INSTANTIATE_KIND(22)
INGOT_INSTANTIATE_FUSED(17, 8)
