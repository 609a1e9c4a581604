// w8a16_gemm.hip - W8A16 (bf16 activations x e4m3 weights) for profiles of
// 65..128 rows, as an LDS-tiled GEMM.
//
// At 128 rows every weight byte feeds 128 rows of MFMA work. A block of 8
// waves (two per SIMD, so one wave's LDS reads overlap the other's MFMAs)
// owns a 128-row x BN-column output tile over one K-slice, as a 4 x 2 grid
// of 32 x BN/2 wave tiles. Each 128-deep k-step needs the activation tile
// (128 rows x 128 bf16 = 32 KiB, an L2 hit: every block reads the same x)
// and BN / 16 weight tiles (e4m3, 2 KiB each, copied verbatim from the
// pre-swizzled region; HBM). Both go global -> LDS with global_load_lds
// (no registers held by bytes in flight), in two rings:
//
//   waves 0-3 load activation stages, NSA deep (L2 latency is short);
//   waves 4-7 load weight stages, NSB deep (HBM latency is long).
//
// A wave's load counter completes in issue order, so one wave issuing both
// would wait for its older weight stages whenever it waits for an
// activation stage; split by wave, each waits only for its own ring. One
// block barrier per k-step then publishes both stages to all waves. Each
// wave reads its activation fragments and weight tiles from LDS, converts
// the weights to bf16 in registers (exact) and issues 16x16x32 bf16 MFMAs.
//
// Activation LDS layout: row r (256 bytes = 16 chunks of 16 bytes) keeps
// logical chunk c at chunk c ^ chunk_swizzle(r), so the 16 lanes of a
// fragment read (16 rows, one logical chunk) hit distinct banks. A load
// instruction (1 KiB) covers 4 rows; lane l writes row 4q + l / 16, physical
// chunk l % 16, so it fetches logical chunk (l % 16) ^ chunk_swizzle(row). Rows past the live M fetch
// the last live row (their results are never stored).
//
// K order inside a k-step: lane (g, r) of a packed weight tile holds column
// r, k = 32 g .. 32 g + 31 (two 1 KiB halves). MFMA j (0..3) of the step
// takes k = 32 g + 8 j .. + 7 from each lane of the A and the B fragment -
// any permutation of K is valid when both operands follow it - so the A
// fragment of MFMA j reads logical chunk 4 g + j of its row.
//
// Split-K (S = gridDim.x / column blocks > 1): fp32 partial fragments to the
// workspace with agent-scope stores, an arrival counter per column block,
// the last block to arrive sums the S slices in slice order and runs the
// epilogue, then resets the counter (as the column-group form of w8a16.hip).
// Nothing waits on another block, so nothing can hang.
//
// Included after w8a16.hip (its weight_fragment), in the one translation unit.
#include "device_common.h"
#include "w8a8_v3.h"

namespace w16g {

template <int BN, int WGM, int WGN, int NSA, int NSB>
struct Tile {
  static constexpr int kBM = 128, kWgm = WGM, kWgn = WGN, kWaves = WGM * WGN;
  static constexpr int kWaveM = kBM / kWgm, kWaveN = BN / kWgn;
  static constexpr int kFM = kWaveM / 16, kFN = kWaveN / 16;
  static constexpr int kAStage = kBM * 256;  // bytes
  static constexpr int kBStage = BN * 128;
  static constexpr int kSmem = NSA * kAStage + NSB * kBStage;
  static constexpr int kLoaders = kWaves / 2;              // waves per ring
  static constexpr int kAIns = kAStage / 1024 / kLoaders;  // per loader wave
  static constexpr int kBIns = kBStage / 1024 / kLoaders;
  static_assert(kSmem + 16 <= 160 * 1024, "LDS budget");
  static_assert(kBStage % (1024 * kLoaders) == 0, "weight half-tiles split evenly");
  static_assert(kFN % 2 == 0, "gate/up pairs a wave's fragments");
  static_assert(NSA >= 2 && NSB >= 2, "rings of at least two stages");
  static_assert((NSA - 2) * kAIns < 64 && (NSB - 2) * kBIns < 64, "vmcnt range");
};

// Waits until at most `later` groups of N load instructions, issued by this
// wave after the group needed, are outstanding; `later` is wave-uniform and
// within 0..D (D = ring depth - 2).
template <int N, int D>
LF_DEVICE void wait_ring(int later) {
  if constexpr (D > 0) {
    if (later >= D) {
      w8a8v3::wait_vmcnt<D * N>();
      return;
    }
    wait_ring<N, D - 1>(later);
  } else {
    w8a8v3::wait_vmcnt<0>();
  }
}

// MODE 0: dense, 1: QKV (three weights, packed Q|K|V output), 2: gate/up
// (each wave column's fragments: kFN / 2 gate tiles, then the up tiles of the
// same h-columns, so SwiGLU pairs fragment j with j + kFN / 2 in a lane).
template <int BN, int WGM, int WGN, int NSA, int NSB, int MODE>
__device__ __forceinline__ void w8a16_gemm_kernel(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                                  const uint8_t *w1, const uint8_t *w2, uint16_t *y,
                                  uint8_t *ws) {
  using T = Tile<BN, WGM, WGN, NSA, NSB>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::kSmem];
  __shared__ int last_block;
  if (!dense_regions_ok<MODE>(w0, w1, w2)) return;
  const WeightHeader &h0 = header_of(w0);
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int nq = static_cast<int>(h0.rows);
  const int nk = MODE == 1 ? static_cast<int>(header_of(w1).rows) : 0;
  // output columns: ld; a block covers BN weight columns (gate/up: BN / 2
  // h-columns)
  const int ld = MODE == 1 ? nq + nk + static_cast<int>(header_of(w2).rows) : nq;
  const int blocks_n = MODE == 2 ? ld / (BN / 2) : ld / BN;
  if (blocks_n < 1) return;
  const int S = static_cast<int>(gridDim.x) / blocks_n;
  if (S < 1) return;  // the geometry rules this out
  const int cb = static_cast<int>(blockIdx.x) / S;
  const int s = static_cast<int>(blockIdx.x) - cb * S;
  const int kt0 = (KT * s) / S, kt1 = (KT * (s + 1)) / S;
  if (cb >= blocks_n || kt1 <= kt0) return;
  const int M = live_rows(counts, T::kBM);
  if (M == 0) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;
  const int g = lane >> 4, r = lane & 15;
  const bool a_loader = wave < T::kLoaders;
  const int lw = a_loader ? wave : wave - T::kLoaders;  // index among its ring's loaders

  // Block slot sl (16 weight columns) -> (region, tile index in it, output
  // column of the slot's first column).
  auto slot = [&](int sl, const uint8_t *&region, int &tile, int &ocol) {
    if constexpr (MODE == 2) {
      const int sw = sl / T::kFN, f = sl % T::kFN;
      const bool up = f >= T::kFN / 2;
      ocol = cb * (BN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN / 2 : f);
      region = up ? w1 : w0;
      tile = ocol >> 4;
    } else {
      ocol = cb * BN + 16 * sl;
      region = w0;
      tile = ocol >> 4;
      if constexpr (MODE == 1) {
        if (ocol >= nq + nk) {
          region = w2;
          tile = (ocol - nq - nk) >> 4;
        } else if (ocol >= nq) {
          region = w1;
          tile = (ocol - nq) >> 4;
        }
      }
    }
  };

  // This lane's channel scales (one per fragment column), requested first.
  float sc[T::kFN];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    int tile, ocol;
    slot(wn * T::kFN + j, region, tile, ocol);
    sc[j] = expert_scales(region, 0)[tile * 16 + r];
  }

  // Global sources of this lane's load instructions at k-tile 0: activation
  // rows for waves 0-3, weight half-tiles for waves 4-7.
  const uint8_t *a_src[T::kAIns];
  const uint8_t *b_src[T::kBIns];
  if (a_loader) {
#pragma unroll
    for (int q = 0; q < T::kAIns; ++q) {
      const int row = 4 * (lw * T::kAIns + q) + (lane >> 4);
      const int src = row < M ? row : M - 1;
      const int chunk = (lane & 15) ^ chunk_swizzle(row);
      a_src[q] = reinterpret_cast<const uint8_t *>(x + static_cast<uint64_t>(src) * K) + chunk * 16;
    }
  } else {
#pragma unroll
    for (int q = 0; q < T::kBIns; ++q) {
      const int hq = lw * T::kBIns + q;
      const uint8_t *region;
      int tile, ocol;
      slot(hq >> 1, region, tile, ocol);
      b_src[q] = expert_tiles(region, 0) + static_cast<uint64_t>(tile) * KT * kTileBytes +
                 (hq & 1) * 1024 + lane * 16;
    }
  }

  const uint32_t smem_base = __builtin_amdgcn_readfirstlane(w8a8v3::lds_offset_of(smem));
  const uint32_t b_base = smem_base + NSA * T::kAStage;
  // Stage i (k-tile kt0 + i) into its ring slot.
  auto issue_a = [&](int i) {
    const uint32_t dst = smem_base + (i % NSA) * T::kAStage + lw * T::kAIns * 1024;
#pragma unroll
    for (int q = 0; q < T::kAIns; ++q) {
      w8a8v3::dma16(a_src[q] + (kt0 + i) * 256, dst + q * 1024);
    }
  };
  auto issue_b = [&](int i) {
    const uint32_t dst = b_base + (i % NSB) * T::kBStage + lw * T::kBIns * 1024;
#pragma unroll
    for (int q = 0; q < T::kBIns; ++q) {
      w8a8v3::dma16(b_src[q] + static_cast<uint64_t>(kt0 + i) * kTileBytes, dst + q * 1024);
    }
  };

  f32x4 acc[T::kFM][T::kFN];
#pragma unroll
  for (int i = 0; i < T::kFM; ++i)
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nkt = kt1 - kt0;
  if (a_loader) {
    for (int i = 0; i < NSA - 1 && i < nkt; ++i) issue_a(i);
  } else {
    for (int i = 0; i < NSB - 1 && i < nkt; ++i) issue_b(i);
  }
  for (int k = 0; k < nkt; ++k) {
    // This wave's part of stage k has landed once at most the later stages
    // it has in flight are outstanding (its loads complete in issue order).
    if (a_loader) {
      wait_ring<T::kAIns, NSA - 2>(nkt - 1 - k);
    } else {
      wait_ring<T::kBIns, NSB - 2>(nkt - 1 - k);
    }
    __syncthreads();  // both stages of k-step k are in LDS, and the slots
                      // refilled below are no longer being read
    if (a_loader) {
      if (k + NSA - 1 < nkt) issue_a(k + NSA - 1);
    } else {
      if (k + NSB - 1 < nkt) issue_b(k + NSB - 1);
    }
    const uint8_t *a = smem + (k % NSA) * T::kAStage;
    const uint8_t *b = smem + NSA * T::kAStage + (k % NSB) * T::kBStage;
    uint4 bq[T::kFN][2];
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) {
      const uint8_t *tile = b + (wn * T::kFN + j) * kTileBytes;
      bq[j][0] = *reinterpret_cast<const uint4 *>(tile + lane * 16);
      bq[j][1] = *reinterpret_cast<const uint4 *>(tile + 1024 + lane * 16);
    }
    bf16x8 af[4][T::kFM];
#pragma unroll
    for (int step = 0; step < 4; ++step)
#pragma unroll
      for (int i = 0; i < T::kFM; ++i) {
        const int row = wm * T::kWaveM + i * 16 + r;
        af[step][i] =
            *reinterpret_cast<const bf16x8 *>(a + row * 256 + ((((g << 2) | step) ^ chunk_swizzle(r)) << 4));
      }
#pragma unroll
    for (int step = 0; step < 4; ++step) {
#pragma unroll
      for (int j = 0; j < T::kFN; ++j) {
        const bf16x8 bf = weight_fragment(bq[j], step);
#pragma unroll
        for (int i = 0; i < T::kFM; ++i) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[step][i], bf, acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // Epilogue. Lane element (i, j, e) is row wm * kWaveM + 16 i + 4 g + e of
  // slot column 16 (wn kFN + j) + r.
  auto store = [&](const f32x4 (&v)[T::kFM][T::kFN]) {
#pragma unroll
    for (int i = 0; i < T::kFM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = wm * T::kWaveM + 16 * i + 4 * g + e;
        if (m >= M) continue;
        if constexpr (MODE == 2) {
#pragma unroll
          for (int j = 0; j < T::kFN / 2; ++j) {
            const uint8_t *region;
            int tile, ocol;
            slot(wn * T::kFN + j, region, tile, ocol);
            const float out = silu_mul(v[i][j][e] * sc[j],
                                       v[i][j + T::kFN / 2][e] * sc[j + T::kFN / 2]);
            y[static_cast<uint64_t>(m) * ld + ocol + r] = static_cast<uint16_t>(f32_to_bf16(out));
          }
        } else {
#pragma unroll
          for (int j = 0; j < T::kFN; ++j) {
            const uint8_t *region;
            int tile, ocol;
            slot(wn * T::kFN + j, region, tile, ocol);
            y[static_cast<uint64_t>(m) * ld + ocol + r] =
                static_cast<uint16_t>(f32_to_bf16(v[i][j][e] * sc[j]));
          }
        }
      }
  };
  if (S == 1) {
    store(acc);
    return;
  }

  // Split-K exchange: fragment ((s * blocks_n + cb) * 8 + wave) * kFM * kFN
  // + i * kFN + j, 256 floats, element e of lane l at e * 64 + l; then one
  // arrival counter per column block. Fragments of rows wholly past M are
  // neither stored nor loaded.
  constexpr int kFrags = T::kFM * T::kFN;
  float *part = reinterpret_cast<float *>(ws);
  int *arrivals = reinterpret_cast<int *>(
      ws + align256(static_cast<uint64_t>(S) * blocks_n * T::kWaves * kFrags * 256 * sizeof(float)));
  auto frag_at = [&](int slice, int i, int j) -> float * {
    return part + ((static_cast<uint64_t>(slice) * blocks_n + cb) * T::kWaves + wave) * kFrags * 256 +
           (i * T::kFN + j) * 256 + lane;
  };
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) {
    if (wm * T::kWaveM + 16 * i + 4 * g < M) {
#pragma unroll
      for (int j = 0; j < T::kFN; ++j) {
        float *p = frag_at(s, i, j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          __hip_atomic_store(p + 64 * e, acc[i][j][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before =
        __hip_atomic_fetch_add(arrivals + cb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before == S - 1;
    if (last) __hip_atomic_store(arrivals + cb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_block = last ? 1 : 0;
  }
  __syncthreads();
  if (last_block == 0) return;
  f32x4 sum[T::kFM][T::kFN];
#pragma unroll
  for (int i = 0; i < T::kFM; ++i)
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) sum[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int slice = 0; slice < S; ++slice) {
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
      const bool live = wm * T::kWaveM + 16 * i + 4 * g < M;
#pragma unroll
      for (int j = 0; j < T::kFN; ++j) {
        f32x4 v = acc[i][j];
        if (slice != s && live) {
          const float *p = frag_at(slice, i, j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = __hip_atomic_load(p + 64 * e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        sum[i][j] += v;
      }
    }
  }
  store(sum);
}

}  // namespace w16g

extern "C" {

// Symbols: lf_fp8_w8a16_{op}_m128_n{BN}; the launch geometry picks BN and the
// K split S (grid = column blocks x S; blocks of 64 WGM WGN threads).
#define LF_W16_GEMM_ENTRIES(BN, WGM, WGN, NSA, NSB)                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_dense_m128_n##BN(               \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) {     \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 0>(counts, x, w, w, w, y, ws);                \
  }                                                                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_qkv_m128_n##BN(                 \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,            \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                             \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 1>(counts, x, wq, wk, wv, y, ws);             \
  }                                                                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_gate_up_m128_n##BN(             \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      uint16_t *h, uint8_t *ws) {                                                                \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 2>(counts, x, wg, wu, wu, h, ws);             \
  }

LF_W16_GEMM_ENTRIES(64, 4, 2, 4, 2)
LF_W16_GEMM_ENTRIES(128, 4, 2, 2, 4)

}  // extern "C"
