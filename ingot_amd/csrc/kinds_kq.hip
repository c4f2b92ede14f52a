// Per-format kernels (see kind_launch.h): GGML types 10 13.
#include "kind_launch.cuh"

INGOT_INSTANTIATE_KIND(10)
INGOT_INSTANTIATE_KIND(13)
INGOT_INSTANTIATE_F16(13)
