// projection.hip - gfx950 kernels of the prefill regime: the per-token
// activation quantizer and the W8A8 FP8 MFMA GEMM (QKV, output/down,
// gate/up + SwiGLU). Entry points and operand lists are documented in
// include/lunaflux_fp8.h; every parameter is a device region.
#include "w8a8_core.h"

namespace {

// ---------------------------------------------------------------------------
// Row quantizer: one block per row. For each span of columns (the whole row
// when group == 0, else `group` columns): amax over the span, ratio = 448 /
// amax (correctly rounded division), codes = e4m3_rne_sat(x * ratio),
// scale = amax / 448 (one per span, in order). An all-zero span gets zero
// codes and scale 0.
// ---------------------------------------------------------------------------
__device__ void quantize_row(const uint16_t *src_row, int K, int group, uint8_t *dst_row,
                             float *scales_row) {
  __shared__ float partial[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int span = group > 0 ? group : K;
  for (int s0 = 0; s0 < K; s0 += span) {
    const uint4 *src = reinterpret_cast<const uint4 *>(src_row + s0);
    const int chunks = span >> 3;  // 8 bf16 per 16-byte chunk
    float amax = 0.0f;
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
      const uint4 v = src[c];
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(w4[i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(w4[i] >> 16)));
      }
    }
    amax = wave_max(amax);
    if (lane == 0) partial[wave] = amax;
    __syncthreads();
    amax = partial[0];
    for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) amax = fmaxf(amax, partial[i]);
    __syncthreads();  // partial[] is reused by the next span
    const bool zero = amax == 0.0f;
    const float ratio = zero ? 0.0f : 448.0f / amax;
    uint2 *dst = reinterpret_cast<uint2 *>(dst_row + s0);
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
      const uint4 v = src[c];
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
      uint32_t out[2] = {0u, 0u};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = zero ? 0u : e4m3_encode(bf16_to_f32(w4[i] & 0xffffu) * ratio);
        const uint32_t hi = zero ? 0u : e4m3_encode(bf16_to_f32(w4[i] >> 16) * ratio);
        out[i >> 1] |= (lo | (hi << 8)) << (16 * (i & 1));
      }
      dst[c] = make_uint2(out[0], out[1]);
    }
    if (threadIdx.x == 0) scales_row[s0 / span] = zero ? 0.0f : amax / 448.0f;
  }
}

__device__ void act_quant_rows(const int32_t *counts, const uint16_t *x, const uint8_t *w,
                               uint8_t *xq) {
  const WeightHeader &h = header_of(w);
  if (h.magic != kWeightMagic) return;
  const int K = static_cast<int>(h.columns);
  const int M = live_rows(counts, 1 << 30);
  const int row = blockIdx.x;
  if (row >= M) return;
  float *scales = reinterpret_cast<float *>(xq + align256(static_cast<uint64_t>(M) * K));
  quantize_row(x + static_cast<uint64_t>(row) * K, K, 0, xq + static_cast<uint64_t>(row) * K,
               scales + row);
}

// ---------------------------------------------------------------------------
// Dense W8A8 GEMM: xq [M, K] e4m3 with per-token scales (the quantizer's
// output) x weights with per-channel scales. MODE 0: dense, 1: qkv (three
// weights, packed Q|K|V columns), 2: gate/up with the SwiGLU epilogue (each
// wave takes 32 h-columns: gate and up tiles of the same columns).
// ---------------------------------------------------------------------------
template <int MODE>
__device__ void w8a8_kernel(const int32_t *counts, const uint8_t *xq, const uint8_t *w0,
                            const uint8_t *w1, const uint8_t *w2, uint16_t *y) {
  __shared__ __attribute__((aligned(16))) uint8_t As[2][w8a8::kAStage];
  const WeightHeader &h0 = header_of(w0);
  if (h0.magic != kWeightMagic) return;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int M = live_rows(counts, 1 << 30);
  const int m0 = blockIdx.y * w8a8::kBM;
  if (m0 >= M) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint8_t *strip[4];
  const float *wscale[4];
  int scol[4];  // column inside its weight (scale index)
  int ocol[4];  // output column
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

  const int arow = tid >> 1;
  const bool arow_live = m0 + arow < M;
  const uint4 *asrc = reinterpret_cast<const uint4 *>(
      xq + static_cast<uint64_t>(m0 + (arow_live ? arow : 0)) * K + (tid & 1) * 64);
  const float *const no_scale[4] = {nullptr, nullptr, nullptr, nullptr};
  f32x4 acc[4][4];
  w8a8::mainloop<false>(asrc, arow_live, strip, KT, As, nullptr, no_scale, acc);

  const float *ascale = reinterpret_cast<const float *>(xq + align256(static_cast<uint64_t>(M) * K));
  const int r = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int m = m0 + w8a8::acc_row(wm, i, lane, rr);
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
                                                             const uint8_t *w, uint8_t *xq) {
  act_quant_rows(counts, x, w, xq);
}

__global__ __launch_bounds__(256) void lf_fp8_w8a8_dense(const int32_t *counts,
                                                         const uint8_t *xq, const uint8_t *w,
                                                         uint16_t *y) {
  w8a8_kernel<0>(counts, xq, w, w, w, y);
}

__global__ __launch_bounds__(256) void lf_fp8_w8a8_qkv(const int32_t *counts,
                                                       const uint8_t *xq, const uint8_t *wq,
                                                       const uint8_t *wk, const uint8_t *wv,
                                                       uint16_t *y) {
  w8a8_kernel<1>(counts, xq, wq, wk, wv, y);
}

__global__ __launch_bounds__(256) void lf_fp8_w8a8_gate_up(const int32_t *counts,
                                                           const uint8_t *xq, const uint8_t *wg,
                                                           const uint8_t *wu, uint16_t *h) {
  w8a8_kernel<2>(counts, xq, wg, wu, wu, h);
}

}  // extern "C"
