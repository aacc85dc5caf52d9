#pragma once

// Kernel-argument table of conv2d_small_f32 (conv.hip), shared with the host launcher
// (csrc/hip/ops.cc): patch element k = (c, ky, kx) of a C x KH x KW filter is read at
// input offset offset[k] = (c * H + ky) * W + kx from the patch's top-left corner, after
// bounds-checking row ky and column kx. Plain C types: passed by value.
namespace dk {

constexpr int kSmallPatch = 32;  // patch elements C * KH * KW of the direct kernel
constexpr int kSmallOc = 8;     // output channels per thread

struct SmallConvTable {
  int patch;
  int offset[kSmallPatch];
  int ky[kSmallPatch];
  int kx[kSmallPatch];
};

}  // namespace dk
