// w8a8_core.h - pieces shared by the e4m3 x e4m3 MFMA GEMMs (dense prefill
// in projection.hip, grouped MoE in moe.hip): the MFMA operand fragment and
// the 128-row tile height the MoE sort counts tiles in. The main loops live
// in w8a8_v3.h (128-wide k-steps, 16x16x128 MFMA) and w8a8_v4.h (64-deep
// half-steps, 32x32x64 MFMA).
#pragma once

#include "device_common.h"

namespace w8a8 {

constexpr int kBM = 128;

// One MFMA operand: 32 e4m3 codes per lane (two 16-byte loads).
union Frag8 {
  uint4 h[2];
  i32x8 v;
};

}  // namespace w8a8
