// w8a16.hip - W8A16 (decode regime): bf16 activations x e4m3 weights.
//
// A block owns one 16-column tile of each of its NW weights (NW = 2 for
// gate/up) and splits K across its WAVES waves. Each wave streams its weight
// tiles with two coalesced 1 KiB loads per tile, keeping kInFlight tiles of
// weights outstanding in a register ring so HBM latency is covered, converts
// them to bf16 in registers (exact) and feeds 16x16x32 bf16 MFMAs. The 8 or
// 4 partial tiles are summed in LDS in a fixed wave order (deterministic),
// scaled per channel (plus SwiGLU for gate/up) and stored as bf16.
//
// Activations: for M <= 32 each wave copies its 16*MT x 128 activation slice
// per k-tile into a private LDS slab with coalesced 1 KiB loads (prefetched
// one k-tile ahead) and reads MFMA fragments from there; for larger M the
// fragments are read straight from global memory.
#include "device_common.h"

#ifndef LF_W16_DENSE_IN_FLIGHT
#define LF_W16_DENSE_IN_FLIGHT 4
#endif

namespace {

union Frag16 {
  uint4 u;
  bf16x8 v;
};

constexpr int kSlabStride = 272;  // one 256-byte k-slice row + 16 bytes of pad

// Converts the 8 e4m3 codes of sub-chunk j (k = 32g + 8j .. +8 of this lane)
// to a bf16x8 B fragment.
LF_DEVICE bf16x8 weight_fragment(const uint4 (&t)[2], int j) {
  const uint4 &h = t[j >> 1];
  Frag16 f;
  e4m3x4_to_bf16x4((j & 1) ? h.z : h.x, f.u.x, f.u.y);
  e4m3x4_to_bf16x4((j & 1) ? h.w : h.y, f.u.z, f.u.w);
  return f.v;
}

template <int NW>
LF_DEVICE void load_tiles(const uint8_t *const (&strip)[NW], int kt, int lane, uint4 (&dst)[NW][2]) {
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const u32x4 *t = reinterpret_cast<const u32x4 *>(strip[i] + kt * kTileBytes);
    const u32x4 lo = __builtin_nontemporal_load(t + lane);
    const u32x4 hi = __builtin_nontemporal_load(t + 64 + lane);
    dst[i][0] = make_uint4(lo.x, lo.y, lo.z, lo.w);
    dst[i][1] = make_uint4(hi.x, hi.y, hi.z, hi.w);
  }
}

LF_DEVICE void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// M <= 32: activations staged through this wave's LDS slab.
template <int WAVES, int MT, int NW>
__device__ void accumulate_staged(int M, int K, const uint16_t *__restrict__ x,
                                  const uint8_t *const (&strip)[NW], uint8_t *slab,
                                  f32x4 (&acc)[MT][NW]) {
  constexpr int kInFlight = NW == 1 ? LF_W16_DENSE_IN_FLIGHT : 2;  // k-tiles of weights outstanding
  constexpr int kRows = 16 * MT, kXq = kRows / 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KT = K >> 7;
  const int kt0 = (KT * wave) / WAVES, kt1 = (KT * (wave + 1)) / WAVES;
  const int g = lane >> 4, r = lane & 15;
  const int xrow = lane >> 4, xcol = (lane & 15) * 8;  // coalesced copy mapping
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (kt0 >= kt1) return;

  // Activation and weight loads of k-tile kt are issued together, kInFlight
  // k-tiles ahead of their use. Vector-memory completions are counted in
  // issue order, so waiting for k-tile kt's data never waits for a later
  // k-tile's loads. Loads of 4-row groups wholly past the live M are not
  // issued at all (the branch is wave-uniform).
  uint4 xr[kInFlight][kXq];
  auto load_x = [&](int kt, uint4 (&dst)[kXq]) {
#pragma unroll
    for (int q = 0; q < kXq; ++q) {
      const int row = 4 * q + xrow;
      if (4 * q < M) {
        dst[q] = row < M ? *reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(row) * K + kt * 128 + xcol)
                         : make_uint4(0u, 0u, 0u, 0u);
      } else {
        dst[q] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  uint4 b[kInFlight][NW][2];
#pragma unroll
  for (int d = 0; d < kInFlight; ++d) {
    if (kt0 + d < kt1) {
      load_x(kt0 + d, xr[d]);
      load_tiles<NW>(strip, kt0 + d, lane, b[d]);
    }
  }
  for (int base = kt0; base < kt1; base += kInFlight) {
#pragma unroll
    for (int d = 0; d < kInFlight; ++d) {
      const int kt = base + d;
      if (kt < kt1) {
        wait_lds();  // the previous k-tile's fragment reads are complete
#pragma unroll
        for (int q = 0; q < kXq; ++q) {
          *reinterpret_cast<uint4 *>(slab + (4 * q + xrow) * kSlabStride + xcol * 2) = xr[d][q];
        }
        wait_lds();  // the slab holds k-tile kt
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          Frag16 a[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            a[mt].u = *reinterpret_cast<const uint4 *>(slab + (mt * 16 + r) * kSlabStride + g * 64 + j * 16);
          }
#pragma unroll
          for (int i = 0; i < NW; ++i) {
            const bf16x8 bf = weight_fragment(b[d][i], j);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              acc[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt].v, bf, acc[mt][i], 0, 0, 0);
            }
          }
        }
        if (kt + kInFlight < kt1) {
          load_x(kt + kInFlight, xr[d]);
          load_tiles<NW>(strip, kt + kInFlight, lane, b[d]);
        }
      }
    }
  }
}

// M > 32: activation fragments read straight from global memory (L2).
template <int WAVES, int MT, int NW>
__device__ void accumulate_direct(int M, int K, const uint16_t *__restrict__ x,
                                  const uint8_t *const (&strip)[NW], f32x4 (&acc)[MT][NW]) {
  constexpr int kChunk = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KT = K >> 7;
  const int kt0 = (KT * wave) / WAVES, kt1 = (KT * (wave + 1)) / WAVES;
  const int g = lane >> 4, r = lane & 15;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int base = kt0; base < kt1; base += kChunk) {
    uint4 b[kChunk][NW][2];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (base + c < kt1) load_tiles<NW>(strip, base + c, lane, b[c]);
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (base + c < kt1) {
        const int kt = base + c;
        Frag16 a[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + r;
          const uint4 *p = reinterpret_cast<const uint4 *>(x + static_cast<uint64_t>(m) * K + kt * 128 + g * 32);
#pragma unroll
          for (int j = 0; j < 4; ++j) a[mt][j].u = m < M ? p[j] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int i = 0; i < NW; ++i) {
            const bf16x8 bf = weight_fragment(b[c][i], j);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              acc[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt][j].v, bf, acc[mt][i], 0, 0, 0);
            }
          }
        }
      }
    }
  }
}

template <int WAVES, int MT, int NW, bool STAGED>
struct W16Shared {
  static constexpr int kSlabBytes = STAGED ? WAVES * 16 * MT * kSlabStride : 0;
  static constexpr int kRedBytes = WAVES * MT * NW * 64 * 16;
  static constexpr int kBytes = kSlabBytes > kRedBytes ? kSlabBytes : kRedBytes;
};

// MODE 0: dense, 1: qkv (three weights, packed Q|K|V output), 2: gate/up.
template <int WAVES, int MT, int MODE>
__device__ void w8a16_kernel(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                             const uint8_t *w1, const uint8_t *w2, uint16_t *y) {
  constexpr int NW = MODE == 2 ? 2 : 1;
  constexpr bool STAGED = MT <= 2;
  using Shared = W16Shared<WAVES, MT, NW, STAGED>;
  // The activation slabs and the reduction buffer share this storage; a
  // block barrier separates their lifetimes.
  __shared__ __attribute__((aligned(16))) uint8_t smem[Shared::kBytes];
  const WeightHeader &h0 = header_of(w0);
  if (h0.magic != kWeightMagic) return;
  const int K = static_cast<int>(h0.columns);
  const int M = live_rows(counts, 16 * MT);
  int tile = blockIdx.x;
  const int out_col0 = tile * 16;
  int ld = static_cast<int>(h0.rows);
  const uint8_t *region[NW];
  region[0] = w0;
  if (MODE == 1) {
    const int tq = static_cast<int>(h0.rows) >> 4;
    const int tk = static_cast<int>(header_of(w1).rows) >> 4;
    ld = static_cast<int>(h0.rows + header_of(w1).rows + header_of(w2).rows);
    if (tile >= tq + tk) {
      region[0] = w2;
      tile -= tq + tk;
    } else if (tile >= tq) {
      region[0] = w1;
      tile -= tq;
    }
  }
  if (NW == 2) region[NW - 1] = w1;
  const uint8_t *strip[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    strip[i] = expert_tiles(region[i], 0) + static_cast<uint64_t>(tile) * (K >> 7) * kTileBytes;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  f32x4 acc[MT][NW];
  if constexpr (STAGED) {
    accumulate_staged<WAVES, MT, NW>(M, K, x, strip, smem + wave * 16 * MT * kSlabStride, acc);
    __syncthreads();  // every slab is dead before the reduction buffer reuses it
  } else {
    accumulate_direct<WAVES, MT, NW>(M, K, x, strip, acc);
  }
  f32x4(*red)[MT * NW][64] = reinterpret_cast<f32x4(*)[MT * NW][64]>(smem);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) red[wave][mt * NW + i][lane] = acc[mt][i];
  __syncthreads();

  const float *scale0 = expert_scales(region[0], 0);
  const float *scale1 = expert_scales(region[NW - 1], 0);
  for (int e = threadIdx.x; e < MT * 256; e += blockDim.x) {
    const int mt = e >> 8, row16 = (e >> 4) & 15, c = e & 15;
    const int m = mt * 16 + row16;
    if (m >= M) continue;
    const int src_lane = (row16 >> 2) * 16 + c, rr = row16 & 3;
    float s[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      float v = 0.0f;
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) v += red[wv][mt * NW + i][src_lane][rr];
      s[i] = v;
    }
    const int n_local = tile * 16 + c;
    const float out = MODE == 2 ? silu_mul(s[0] * scale0[n_local], s[NW - 1] * scale1[n_local])
                                : s[0] * scale0[n_local];
    y[static_cast<uint64_t>(m) * ld + out_col0 + c] = static_cast<uint16_t>(f32_to_bf16(out));
  }
}

}  // namespace

#ifndef LF_W16_DENSE_WAVES
#define LF_W16_DENSE_WAVES 8
#endif
#ifndef LF_W16_GATE_UP_WAVES
#define LF_W16_GATE_UP_WAVES 4
#endif

extern "C" {

#define LF_W8A16_ENTRIES(MT, M)                                                              \
  __global__ __launch_bounds__(LF_W16_DENSE_WAVES * 64) void lf_fp8_w8a16_dense_m##M(        \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y) {             \
    w8a16_kernel<LF_W16_DENSE_WAVES, MT, 0>(counts, x, w, w, w, y);                          \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16_DENSE_WAVES * 64) void lf_fp8_w8a16_qkv_m##M(          \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,        \
      const uint8_t *wv, uint16_t *y) {                                                      \
    w8a16_kernel<LF_W16_DENSE_WAVES, MT, 1>(counts, x, wq, wk, wv, y);                       \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16_GATE_UP_WAVES * 64) void lf_fp8_w8a16_gate_up_m##M(    \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,        \
      uint16_t *h) {                                                                         \
    w8a16_kernel<LF_W16_GATE_UP_WAVES, MT, 2>(counts, x, wg, wu, wu, h);                     \
  }

LF_W8A16_ENTRIES(1, 16)
LF_W8A16_ENTRIES(2, 32)
LF_W8A16_ENTRIES(4, 64)
LF_W8A16_ENTRIES(8, 128)

}  // extern "C"
