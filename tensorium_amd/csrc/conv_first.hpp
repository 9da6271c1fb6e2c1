// The network's first convolution (C <= 4 channels, NCHW image in,
// channels-last out) on the matrix cores (conv_first.hip).
#pragma once
#include "conv_args.hpp"

namespace tnh {
namespace conv {

// Whether launch_first_mfma serves this call: 3x3 over an NCHW image (the
// caller checks), 1 <= C <= 4, F <= 64 with F % 4 == 0, no residual, a
// 16-byte aligned channels-last output with outPix % 4 == 0, no epilogue
// variant.
bool first_mfma_ok(const ConvArgs& a);
int launch_first_mfma(const ConvArgs& a, hipStream_t s);

}  // namespace conv
}  // namespace tnh
