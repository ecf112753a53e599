// Small-window convolutions (conv_small.hip): layers whose window holds at
// most 32 elements (C*kh*kw <= 32) and whose output has at most 64 channels,
// the 3-channel first layer of configs 4/5. Internal to the library.
#pragma once

#include "common.h"

namespace vkhip {

// Whether win_conv_forward takes this forward convolution (oh x ow outputs
// per image, weights [Cout][C*kh*kw] described by wd).
bool win_fwd_fits(const vkhip_operand& xd, const vkhip_unfold& pr, uint32_t channels, uint64_t ck,
                  uint32_t cout, const vkhip_operand& wd, uint32_t oh, uint32_t ow);

// out[n][co][p] = relu?(sum_j w[co][j] * window_j(x[n], p) + bias[co]): the
// implicit-im2col GEMM's bits (same K pairing and order), plus the epilogue's
// one rounded add.
int win_conv_forward(const float* x, const vkhip_operand& xd, const float* w, const vkhip_operand& wd,
                     float* out, const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout,
                     uint32_t ck, uint32_t oh, uint32_t ow, const float* bias, int64_t bias_stride,
                     bool relu);

// Whether win_conv_weight_grad_sum takes this batch-summed weight gradient
// (gradient [N][Cout][oh*ow] described by gd).
bool win_wgrad_fits(const float* g, const vkhip_operand& gd, const vkhip_operand& xd, const vkhip_unfold& pr,
                    uint32_t channels, uint64_t ck, uint32_t cout, uint64_t batch, uint32_t oh, uint32_t ow);

// dW[co][j] = sum over n, p of g[n][co][p] * window_j(x[n], p): workgroup
// partials, then their fold in a fixed order (two launches).
int win_conv_weight_grad_sum(const float* x, const vkhip_operand& xd, const float* g, const vkhip_operand& gd,
                             float* out, const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout,
                             uint32_t ck, uint32_t oh, uint32_t ow);

// Whether win_conv_pool_weight_bias_grad takes this layer: y [N][Cout][oh][ow]
// (described by yd as the gradient is for win_wgrad_fits) and its 2x2,
// stride-2 max-pool's output gradient gp (image and channel strides gpsn,
// gpsc; rows contiguous), with ow in {4, 8, 16, 32}, oh even, N*oh*ow a power
// of two.
bool win_pool_wgrad_fits(const float* y, const vkhip_operand& yd, const float* gp, int64_t gpsn, int64_t gpsc,
                         const vkhip_operand& xd, const vkhip_unfold& pr, uint32_t channels, uint64_t ck,
                         uint32_t cout, uint64_t batch, uint32_t oh, uint32_t ow);

// The conv layer's weight and bias gradients from its pool's output gradient:
// dz = the max-pool backward of gp over y masked by the relu (y <= 0 -> 0),
// formed in the kernel and never written; out [Cout][K] = the batch-summed
// weight gradient of dz (win_conv_weight_grad_sum's bits) and bias_out[Cout]
// = the sum of dz over N, oh, ow in the pairwise tree's order (the
// reduction's bits). Two launches.
int win_conv_pool_weight_bias_grad(const float* x, const vkhip_operand& xd, const float* y, const vkhip_operand& yd,
                                   const float* gp, int64_t gpsn, int64_t gpsc, float* out, float* bias_out,
                                   const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout,
                                   uint32_t ck, uint32_t oh, uint32_t ow);

// Whether win_conv_input_grad takes this input gradient (unit strides, C*kh*kw
// <= 32, Cout <= 128).
bool win_dx_fits(const vkhip_operand& gd, int64_t w_row, const vkhip_unfold& pr, uint32_t batch, uint32_t channels,
                 uint32_t cout, uint32_t oh, uint32_t ow);

// dX = col2im(flat_weight^T @ grad) in one launch, the reference lowering's
// bits; grad [N][Cout][oh][ow] with contiguous positions, the flat weight
// [Cout][C*kh*kw] with row stride w_row.
int win_conv_input_grad(const float* g, const vkhip_operand& gd, const float* w, int64_t w_row, float* out,
                        const vkhip_unfold& pr, uint32_t batch, uint32_t channels, uint32_t cout, uint32_t oh,
                        uint32_t ow);

}  // namespace vkhip
