// kernels.hpp -- internal launchers shared between translation units.
#pragma once

#include <cstdint>

struct NeuralTensor;

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

// Gradient clipping over a tensor list (NULL entries skipped): the global-norm
// clip (total_norm, when non-null, receives the pre-clip norm) and the value
// clip.  Both run on the active stream; see clip.hip.
int clip_norm_list(NeuralTensor *const *grads, int64_t count, double max_norm, double *total_norm);
int clip_value_list(NeuralTensor *const *grads, int64_t count, double lo, double hi);

}  // namespace nh
