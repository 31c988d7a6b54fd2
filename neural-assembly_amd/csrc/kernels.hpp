// kernels.hpp -- internal launchers shared between translation units.
#pragma once

#include <cstdint>

namespace nh {

// Contiguous fill of n elements (f32 stores (float)value).
int launch_fill(void *dst, int dtype, int64_t n, double value);
// Fill every element addressed by shape / byte strides.
int launch_fill_strided(void *dst, int dtype, const int64_t *shape, const int64_t *bstride, int ndim,
                        double value);
// Copy src -> dst in logical row-major order (equal element counts, any
// shapes/byte strides, element size es).
int launch_copy_nd(void *dst, const int64_t *dshape, const int64_t *dstride, int dndim, const void *src,
                   const int64_t *sshape, const int64_t *sstride, int sndim, int es);

}  // namespace nh
