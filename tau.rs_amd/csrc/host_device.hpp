// TAU_HOST_DEVICE marks index and arithmetic helpers that the kernels use and
// that host-side checks compile unchanged with a plain C++ compiler.
#pragma once

#if defined(__HIPCC__)
#define TAU_HOST_DEVICE __host__ __device__
#else
#define TAU_HOST_DEVICE
#endif
