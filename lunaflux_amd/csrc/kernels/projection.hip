// projection.hip - gfx950 kernels of the prefill regime: the per-token
// activation quantizer and the W8A8 FP8 MFMA GEMM (QKV, output/down,
// gate/up + SwiGLU). Entry points and operand lists are documented in
// include/lunaflux_fp8.h; every parameter is a device region.
#include "device_common.h"

namespace {

// ---------------------------------------------------------------------------
// Per-token activation quantizer (prefill prologue).
// One block per row: amax over the row, ratio = 448 / amax (correctly
// rounded division), codes = e4m3_rne_sat(x * ratio), scale = amax / 448.
// An all-zero row gets zero codes and scale 0.
// ---------------------------------------------------------------------------
__device__ void act_quant_rows(const int32_t *counts, const uint16_t *x,
                               const uint8_t *w, uint8_t *xq) {
  const WeightHeader &h = header_of(w);
  if (h.magic != kWeightMagic) return;
  const int K = static_cast<int>(h.columns);
  const int M = live_rows(counts, 1 << 30);
  const int row = blockIdx.x;
  if (row >= M) return;
  const uint4 *src = reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(row) * K);
  const int chunks = K >> 3;  // 8 bf16 per 16-byte chunk
  float amax = 0.0f;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    uint4 v = src[c];
    uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      amax = fmaxf(amax, fabsf(bf16_to_f32(w4[i] & 0xffffu)));
      amax = fmaxf(amax, fabsf(bf16_to_f32(w4[i] >> 16)));
    }
  }
  amax = wave_max(amax);
  __shared__ float partial[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) partial[wave] = amax;
  __syncthreads();
  amax = partial[0];
  for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) amax = fmaxf(amax, partial[i]);
  const bool zero = amax == 0.0f;
  const float ratio = zero ? 0.0f : 448.0f / amax;
  uint2 *dst = reinterpret_cast<uint2 *>(xq + static_cast<uint64_t>(row) * K);
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    uint4 v = src[c];
    uint32_t w4[4] = {v.x, v.y, v.z, v.w};
    uint32_t out[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo = zero ? 0u : e4m3_encode(bf16_to_f32(w4[i] & 0xffffu) * ratio);
      uint32_t hi = zero ? 0u : e4m3_encode(bf16_to_f32(w4[i] >> 16) * ratio);
      out[i >> 1] |= (lo | (hi << 8)) << (16 * (i & 1));
    }
    dst[c] = make_uint2(out[0], out[1]);
  }
  if (threadIdx.x == 0) {
    float *scales = reinterpret_cast<float *>(xq + align256(static_cast<uint64_t>(M) * K));
    scales[row] = zero ? 0.0f : amax / 448.0f;
  }
}

// ---------------------------------------------------------------------------
// W8A8: e4m3 activations (per-token scales) x e4m3 weights (per-channel
// scales), prefill regime. Block tile 128 x 128 x 128 (K), 4 waves as 2 x 2,
// each wave 64 x 64 = 4 x 4 tiles of v_mfma_scale_f32_16x16x128_f8f6f4
// (unit block scales). Activations are staged through double-buffered LDS
// with an XOR swizzle of 16-byte chunks; weight fragments are loaded from
// their pre-swizzled tiles straight into registers.
// ---------------------------------------------------------------------------
constexpr int kBM = 128;
constexpr int kAStage = kBM * 128;

union Frag8 {
  uint4 h[2];
  i32x8 v;
};

LF_DEVICE int a_chunk_offset(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

template <int MODE>
__device__ void w8a8_kernel(const int32_t *counts, const uint8_t *xq,
                            const uint8_t *w0, const uint8_t *w1,
                            const uint8_t *w2, uint16_t *y) {
  __shared__ __attribute__((aligned(16))) uint8_t As[2][kAStage];
  const WeightHeader &h0 = header_of(w0);
  if (h0.magic != kWeightMagic) return;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int M = live_rows(counts, 1 << 30);
  const int m0 = blockIdx.y * kBM;
  if (m0 >= M) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Weight fragments of this wave: 4 tiles of 16 columns.
  const uint8_t *strip[4];
  const float *wscale[4];
  int scol[4];   // column inside its weight (scale index)
  int ocol[4];   // output column
  int ld;
  if (MODE == 2) {
    ld = static_cast<int>(h0.rows);
    const int c0 = blockIdx.x * 64 + wn * 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint8_t *reg = j < 2 ? w0 : w1;
      const int col = c0 + (j & 1) * 16;
      strip[j] = expert_tiles(reg, 0) + static_cast<uint64_t>(col >> 4) * KT * kTileBytes;
      wscale[j] = expert_scales(reg, 0);
      scol[j] = col;
      ocol[j] = col;
    }
  } else {
    const int tq = static_cast<int>(h0.rows) >> 4;
    const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
    ld = MODE == 1 ? static_cast<int>(h0.rows + header_of(w1).rows + header_of(w2).rows)
                   : static_cast<int>(h0.rows);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int t = blockIdx.x * 8 + wn * 4 + j;
      ocol[j] = t * 16;
      const uint8_t *reg = w0;
      if (MODE == 1) {
        if (t >= tq + tk) {
          reg = w2;
          t -= tq + tk;
        } else if (t >= tq) {
          reg = w1;
          t -= tq;
        }
      }
      strip[j] = expert_tiles(reg, 0) + static_cast<uint64_t>(t) * KT * kTileBytes;
      wscale[j] = expert_scales(reg, 0);
      scol[j] = t * 16;
    }
  }

  // Activation tile loads: thread t copies row t/2, bytes 64*(t&1) .. +64.
  const int arow = tid >> 1;
  const bool arow_live = m0 + arow < M;
  const uint4 *asrc = reinterpret_cast<const uint4 *>(
      xq + static_cast<uint64_t>(m0 + (arow_live ? arow : 0)) * K + (tid & 1) * 64);
  uint4 ar[4];
  uint4 br[4][2];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ar[c] = arow_live ? asrc[kt * 8 + c] : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      *reinterpret_cast<uint4 *>(&As[buf][a_chunk_offset(arow, (tid & 1) * 4 + c)]) = ar[c];
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

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  load_b(0, br);
  store_a(0);
  __syncthreads();
  const int g = lane >> 4, r = lane & 15;
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

  const float *ascale = reinterpret_cast<const float *>(xq + align256(static_cast<uint64_t>(M) * K));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int m = m0 + wm * 64 + i * 16 + g * 4 + rr;
      if (m >= M) continue;
      const float sa = ascale[m];
      uint16_t *yrow = y + static_cast<uint64_t>(m) * ld;
      if (MODE == 2) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = scol[j] + r;
          const float gv = acc[i][j][rr] * sa * wscale[j][col];
          const float uv = acc[i][j + 2][rr] * sa * wscale[j + 2][col];
          yrow[ocol[j] + r] = static_cast<uint16_t>(f32_to_bf16(silu_mul(gv, uv)));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = acc[i][j][rr] * sa * wscale[j][scol[j] + r];
          yrow[ocol[j] + r] = static_cast<uint16_t>(f32_to_bf16(v));
        }
      }
    }
  }
}

}  // namespace

extern "C" {

__global__ __launch_bounds__(256) void lf_fp8_act_quant_rows(const int32_t *counts,
                                                             const uint16_t *x,
                                                             const uint8_t *w,
                                                             uint8_t *xq) {
  act_quant_rows(counts, x, w, xq);
}

__global__ __launch_bounds__(256) void lf_fp8_w8a8_dense(const int32_t *counts,
                                                         const uint8_t *xq,
                                                         const uint8_t *w,
                                                         uint16_t *y) {
  w8a8_kernel<0>(counts, xq, w, w, w, y);
}

__global__ __launch_bounds__(256) void lf_fp8_w8a8_qkv(const int32_t *counts,
                                                       const uint8_t *xq,
                                                       const uint8_t *wq,
                                                       const uint8_t *wk,
                                                       const uint8_t *wv,
                                                       uint16_t *y) {
  w8a8_kernel<1>(counts, xq, wq, wk, wv, y);
}

__global__ __launch_bounds__(256) void lf_fp8_w8a8_gate_up(const int32_t *counts,
                                                           const uint8_t *xq,
                                                           const uint8_t *wg,
                                                           const uint8_t *wu,
                                                           uint16_t *h) {
  w8a8_kernel<2>(counts, xq, wg, wu, wu, h);
}

}  // extern "C"
