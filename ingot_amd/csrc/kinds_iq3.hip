// Per-format kernels (see kind_launch.h): GGML types 18 21 29.
#include "kind_launch.cuh"

INGOT_INSTANTIATE_KIND(18)
INGOT_INSTANTIATE_KIND(21)
INGOT_INSTANTIATE_KIND(29)
INGOT_INSTANTIATE_FUSED(21, 42)
