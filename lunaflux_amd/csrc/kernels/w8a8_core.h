// w8a8_core.h - the e4m3 x e4m3 MFMA main loop shared by the dense
// (prefill) and grouped (MoE) GEMMs.
//
// Block tile 128 (rows) x 128 (columns) x 128 (K per step), 256 threads as
// 2 x 2 waves, each wave 64 x 64 = 4 x 4 tiles of
// v_mfma_scale_f32_16x16x128_f8f6f4 with unit block scales. Activation rows
// are staged through double-buffered LDS (XOR swizzle of 16-byte chunks, so
// the fragment reads are conflict free); weight fragments come straight from
// their pre-swizzled 16 x 128 tiles into registers, one k-step ahead.
//
// The caller decides which activation row each thread copies (a plain row
// for the dense GEMM, a gathered token row for the grouped GEMM) and which
// weight tiles each wave reads, then applies its own epilogue to acc.
#pragma once

#include "device_common.h"

namespace w8a8 {

constexpr int kBM = 128;
constexpr int kAStage = kBM * 128;

union Frag8 {
  uint4 h[2];
  i32x8 v;
};

LF_DEVICE int a_chunk_offset(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

// Row r of lane l's fragment i, rr: the tile row this accumulator element
// belongs to (wave row wm).
LF_DEVICE int acc_row(int wm, int i, int lane, int rr) { return wm * 64 + i * 16 + (lane >> 4) * 4 + rr; }

// Main loop. Thread t copies tile row t/2, bytes 64*(t%2)..+64 of every
// k-step from `arow` (already offset to that half-row; ignored when
// !arow_live, which stages zeros). Wave (wm, wn) multiplies tile rows
// wm*64..+64 by the 4 weight strips in `strip`.
//
// BLOCK = true applies 128 x 128 block scales inside the loop: after each
// k-step, acc += step * sa[row][kt] * sw[j][kt], where sa_lds holds the
// block's activation scales [kBM][KT] (row-major, staged in LDS by the
// caller) and sw[j] points at fragment j's weight scale row (one per kt).
template <bool BLOCK>
__device__ void mainloop(const uint4 *arow, bool arow_live, const uint8_t *const (&strip)[4],
                         int KT, uint8_t (*As)[kAStage], const float *sa_lds,
                         const float *const (&sw)[4], f32x4 (&acc)[4][4]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1;
  const int trow = tid >> 1, thalf = tid & 1;
  const int g = lane >> 4, r = lane & 15;
  uint4 ar[4];
  uint4 br[4][2];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int c = 0; c < 4; ++c) ar[c] = arow_live ? arow[kt * 8 + c] : make_uint4(0u, 0u, 0u, 0u);
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      *reinterpret_cast<uint4 *>(&As[buf][a_chunk_offset(trow, thalf * 4 + c)]) = ar[c];
    }
  };
  auto load_b = [&](int kt, uint4 (&dst)[4][2]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 *t = reinterpret_cast<const uint4 *>(strip[j] + kt * kTileBytes);
      dst[j][0] = t[lane];
      dst[j][1] = t[64 + lane];
    }
  };
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  load_b(0, br);
  store_a(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    uint4 bn[4][2];
    const bool more = kt + 1 < KT;
    if (more) {
      load_a(kt + 1);
      load_b(kt + 1, bn);
    }
    Frag8 af[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wm * 64 + i * 16 + r;
      af[i].h[0] = *reinterpret_cast<const uint4 *>(&As[cur][a_chunk_offset(row, 2 * g)]);
      af[i].h[1] = *reinterpret_cast<const uint4 *>(&As[cur][a_chunk_offset(row, 2 * g + 1)]);
    }
    if constexpr (BLOCK) {
      f32x4 step[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Frag8 bf;
        bf.h[0] = br[j][0];
        bf.h[1] = br[j][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          step[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              af[i].v, bf.v, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
        }
      }
      float swk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) swk[j] = sw[j][kt];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const float sa = sa_lds[acc_row(wm, i, lane, rr) * KT + kt];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j][rr] += step[i][j][rr] * (sa * swk[j]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Frag8 bf;
        bf.h[0] = br[j][0];
        bf.h[1] = br[j][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              af[i].v, bf.v, acc[i][j], 0, 0, 0, 127, 0, 127);
        }
      }
    }
    if (more) store_a(cur ^ 1);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        br[j][0] = bn[j][0];
        br[j][1] = bn[j][1];
      }
    }
  }
}

}  // namespace w8a8
