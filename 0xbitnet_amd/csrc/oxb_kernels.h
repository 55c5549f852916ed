// Internal include: the public hot-path ABI plus shared launch helpers.
#pragma once
#include "../../include/oxbitnet_ops.h"

extern "C" int oxb_quantize_rows_tiled(const float *x, const float *gamma, float eps, int n_tok,
                                       int D, void *Xt, float *scales, int *sums, void *stream);
