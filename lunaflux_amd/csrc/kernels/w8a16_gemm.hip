// w8a16_gemm.hip - W8A16 (bf16 activations x e4m3 weights) for profiles of
// 65..128 rows, as an LDS-tiled GEMM.
//
// At 128 rows every weight byte feeds 128 rows of MFMA work. A block of 8
// waves (two per SIMD, so one wave's LDS reads overlap the other's MFMAs)
// owns a 128-row x BN-column output tile over one K-slice, as a WGM x WGN
// grid of wave tiles: 2 x 4 tiles of 64 x 32 at BN = 128 (each weight tile
// converted to bf16 by two waves instead of four: down and qkv at 128 rows
// 0.4-1.1 us faster than 4 x 2), 4 x 2 tiles of 32 x 32 at BN = 64 (a wave
// column needs an even count of 16-column fragments for gate/up's pairs).
// Each 128-deep k-step needs the activation tile
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
// The operands sit in two register sets: right after the barrier that
// publishes k-step k + 1, a wave issues that step's LDS reads and then
// runs step k's MFMAs on the other set, so the reads land under the MFMAs
// instead of before them (M = 128 layer 107.4-111.1 -> 106.0-107.0 us,
// GatedMlp 77-81 -> 74-77 us, A/B over eight rounds, bit-identical). The
// compiler places the reads among the MFMAs; pinning all of them ahead of
// the MFMAs measured slower.
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
#include "phases.h"
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
// smem: the block's LDS (T::kSmem bytes, 1 KiB aligned). bid / nblocks: the
// block's index and the block count of this GEMM's part of the grid
// (default blockIdx.x, gridDim.x). gate(s) runs once the weight ring's
// first stages are in flight and before any activation load of K-slice s;
// if it returns false the block waits for its loads into LDS and returns
// (no activation load, no store, no split-K arrival). THROUGH: the outputs
// are stored through the XCD's L2 (phases.h), for an output that blocks of
// the same launch read.
// BLOCK: the weights carry 128 x 128 block scales (s[N/128][K/128]) instead
// of channel scales. A k-step is one 128-deep scale block and a fragment's
// 16 columns lie in one 128-row block, so each k-step's MFMAs accumulate
// into fresh fragments, which are then multiplied by that block's scale
// (one per wave and fragment, a scalar load) and added to the running sums
// (y = sum_kt s[nb][kt] sum_{k in kt} x_k q_k, fp32); the epilogue's
// multiplier is 1.
template <int BN, int WGM, int WGN, int NSA, int NSB, int MODE, bool THROUGH = false, class Gate = NoWait,
          bool BLOCK = false>
__device__ __forceinline__ void w8a16_gemm_kernel(uint8_t *smem, const int32_t *counts, const uint16_t *x,
                                                  const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                                  uint16_t *y, uint8_t *ws, int bid = -1, int nblocks = -1,
                                                  const Gate &gate = Gate{}) {
  using T = Tile<BN, WGM, WGN, NSA, NSB>;
  __shared__ int last_block;
  if (!dense_regions_ok<MODE, BLOCK ? kScaleBlock128 : kScalePerChannel>(w0, w1, w2)) return;
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
  const int nb = nblocks < 0 ? static_cast<int>(gridDim.x) : nblocks;
  const int block = bid < 0 ? static_cast<int>(blockIdx.x) : bid;
  const int S = nb / blocks_n;
  // A grid whose split is not 1..KT (the geometry rules it out) stores
  // nothing in any block: an empty K-slice would never arrive, and its
  // column block's counter would stay raised for later launches.
  if (S < 1 || S > KT) return;
  const int cb = block / S;
  const int s = block - cb * S;
  const int kt0 = (KT * s) / S, kt1 = (KT * (s + 1)) / S;
  if (cb >= blocks_n) return;
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
  // Block scales: the multiplier is 1, and bs[j] points at the k-step
  // scales of fragment j's 128-row block from this slice's first k-tile.
  float sc[T::kFN];
  const float *bs[BLOCK ? T::kFN : 1];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    int tile, ocol;
    slot(wn * T::kFN + j, region, tile, ocol);
    if constexpr (BLOCK) {
      sc[j] = 1.0f;
      bs[j] = reinterpret_cast<const float *>(w8a8v3::uniform_ptr(reinterpret_cast<const uint8_t *>(
          expert_scales(region, 0) + static_cast<uint64_t>(tile >> 3) * KT + kt0)));
    } else {
      sc[j] = expert_scales(region, 0)[tile * 16 + r];
    }
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
  // Step i of the slice runs k-tile kt0 + ktile(i). Unsplit (S == 1): the
  // k-tiles from (block / 8) mod nkt on, wrapping around. Blocks are
  // dispatched to the 8 XCDs in turn, so the column blocks sharing one L2
  // read different k-tiles of x at a time instead of the same few L2
  // channels (gate/up at 128 rows: 1.1-2.0 us less per launch). Split
  // launches keep the plain order: their blocks read disjoint slices, and
  // o at 128 rows (three slices) was 0.2-0.4 us slower rotated.
  const int nkt = kt1 - kt0;
  const int rot = S == 1 ? (block >> 3) % nkt : 0;
  auto ktile = [&](int i) { return i + rot < nkt ? i + rot : i + rot - nkt; };
  // Stage i (k-tile kt0 + ktile(i)) into its ring slot.
  auto issue_a = [&](int i) {
    const uint32_t dst = smem_base + (i % NSA) * T::kAStage + lw * T::kAIns * 1024;
    const int kt = kt0 + ktile(i);
#pragma unroll
    for (int q = 0; q < T::kAIns; ++q) {
      w8a8v3::dma16(a_src[q] + kt * 256, dst + q * 1024);
    }
  };
  auto issue_b = [&](int i) {
    const uint32_t dst = b_base + (i % NSB) * T::kBStage + lw * T::kBIns * 1024;
    const int kt = kt0 + ktile(i);
#pragma unroll
    for (int q = 0; q < T::kBIns; ++q) {
      w8a8v3::dma16(b_src[q] + static_cast<uint64_t>(kt) * kTileBytes, dst + q * 1024);
    }
  };

  f32x4 acc[T::kFM][T::kFN];
#pragma unroll
  for (int i = 0; i < T::kFM; ++i)
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (!a_loader) {
    for (int i = 0; i < NSB - 1 && i < nkt; ++i) issue_b(i);
  }
  if (!gate(s)) {
    w8a8v3::wait_vmcnt<0>();  // no load may land in LDS after the block ends
    return;
  }
  if (a_loader) {
    for (int i = 0; i < NSA - 1 && i < nkt; ++i) issue_a(i);
  }

  // A k-step's operands in registers: the wave's weight tiles (e4m3) and
  // activation fragments, read from the step's LDS stages. Two sets: the
  // next step's are read while this step's MFMAs run.
  struct Frags {
    uint4 bq[T::kFN][2];
    bf16x8 af[4][T::kFM];
  };
  auto read_frags = [&](int k, Frags &f) {
    const uint8_t *a = smem + (k % NSA) * T::kAStage;
    const uint8_t *b = smem + NSA * T::kAStage + (k % NSB) * T::kBStage;
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) {
      const uint8_t *tile = b + (wn * T::kFN + j) * kTileBytes;
      f.bq[j][0] = *reinterpret_cast<const uint4 *>(tile + lane * 16);
      f.bq[j][1] = *reinterpret_cast<const uint4 *>(tile + 1024 + lane * 16);
    }
#pragma unroll
    for (int step = 0; step < 4; ++step)
#pragma unroll
      for (int i = 0; i < T::kFM; ++i) {
        const int row = wm * T::kWaveM + i * 16 + r;
        f.af[step][i] =
            *reinterpret_cast<const bf16x8 *>(a + row * 256 + ((((g << 2) | step) ^ chunk_swizzle(r)) << 4));
      }
  };
  // Stage k + 1 visible to every wave (this wave's part landed: at most the
  // stages it issued after k + 1 are outstanding, its loads completing in
  // issue order), then stage k + NS into the slot of stage k, which every
  // wave read into registers before this barrier.
  auto advance = [&](int k) {
    if (a_loader) {
      wait_ring<T::kAIns, NSA - 2>(nkt - 2 - k);
    } else {
      wait_ring<T::kBIns, NSB - 2>(nkt - 2 - k);
    }
    __syncthreads();
    if (a_loader) {
      if (k + NSA < nkt) issue_a(k + NSA);
    } else {
      if (k + NSB < nkt) issue_b(k + NSB);
    }
  };
  auto compute = [&](int k, const Frags &f) {
    // BLOCK: this k-step's products, scaled into acc after its MFMAs
    f32x4 part[BLOCK ? T::kFM : 1][T::kFN];
    float sb[BLOCK ? T::kFN : 1];
    if constexpr (BLOCK) {
#pragma unroll
      for (int j = 0; j < T::kFN; ++j) sb[j] = bs[j][ktile(k)];
    }
#pragma unroll
    for (int step = 0; step < 4; ++step) {
#pragma unroll
      for (int j = 0; j < T::kFN; ++j) {
        const bf16x8 bf = weight_fragment(f.bq[j], step);
#pragma unroll
        for (int i = 0; i < T::kFM; ++i) {
          if constexpr (BLOCK) {
            part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                f.af[step][i], bf, step == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : part[i][j], 0, 0, 0);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.af[step][i], bf, acc[i][j], 0, 0, 0);
          }
        }
      }
    }
    if constexpr (BLOCK) {
#pragma unroll
      for (int j = 0; j < T::kFN; ++j)
#pragma unroll
        for (int i = 0; i < T::kFM; ++i) {
          acc[i][j] += part[i][j] * sb[j];
          // keeps these reads of the MFMA results in the MFMAs' basic block
          // (a read sunk past a branch has been issued without the wait
          // states an MFMA result needs: w8a16.hip, BLOCK)
          asm volatile("" : "+v"(acc[i][j]));
        }
    }
  };

  // Stage 0: wait, publish, refill the ring's last slot (never read yet),
  // read its operands.
  if (a_loader) {
    wait_ring<T::kAIns, NSA - 2>(nkt - 1);
  } else {
    wait_ring<T::kBIns, NSB - 2>(nkt - 1);
  }
  __syncthreads();
  if (a_loader) {
    if (NSA - 1 < nkt) issue_a(NSA - 1);
  } else {
    if (NSB - 1 < nkt) issue_b(NSB - 1);
  }
  Frags f0, f1;
  read_frags(0, f0);
  // Two k-steps per round, so each register set keeps a fixed name, and no
  // branch around the reads: the barrier's wait for LDS reads then covers
  // the set the round's first MFMAs use, and the next set's 20 reads stay
  // in flight under them (with a path that skips the barrier, the compiler
  // waited for all LDS reads before the first MFMA).
  int k = 0;
  for (; k + 2 < nkt; k += 2) {
    advance(k);
    read_frags(k + 1, f1);
    compute(k, f0);
    advance(k + 1);
    read_frags(k + 2, f0);
    compute(k + 1, f1);
  }
  if (k + 1 < nkt) {
    advance(k);
    read_frags(k + 1, f1);
    compute(k, f0);
    compute(k + 1, f1);
  } else {
    compute(k, f0);
  }

  // Epilogue. Lane element (i, j, e) is row wm * kWaveM + 16 i + 4 g + e of
  // slot column 16 (wn kFN + j) + r.
  auto put = [&](uint16_t *p, float v) {
    const uint16_t bits = static_cast<uint16_t>(f32_to_bf16(v));
    if constexpr (THROUGH) {
      __hip_atomic_store(p, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      *p = bits;
    }
  };
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
            put(y + static_cast<uint64_t>(m) * ld + ocol + r, out);
          }
        } else {
#pragma unroll
          for (int j = 0; j < T::kFN; ++j) {
            const uint8_t *region;
            int tile, ocol;
            slot(wn * T::kFN + j, region, tile, ocol);
            put(y + static_cast<uint64_t>(m) * ld + ocol + r, v[i][j][e] * sc[j]);
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

// ---------------------------------------------------------------------------
// GatedMlp in one launch for profiles of 65..128 rows (model/plan/plan.mbt:
// 47-59; kernels/reference/mlp.mbt:4-39): the grid's first G1 blocks run the
// gate/up GEMM above (GU_BN columns per block, one K-slice) into h in the
// workspace, written through to memory; the other G2 blocks run the down
// GEMM (DN_BN, split S = G2 / (H / DN_BN)) on h. Down blocks start their
// weight ring, then wait (phases.h) until the gate/up blocks that write the
// h columns of their K-slice have counted themselves done: a gate/up block
// (GU_BN / 2 h-columns, within one 128-column k-tile of the down GEMM) adds
// to the counter of the slice holding its k-tile, one 128-byte line per
// slice counter (phases.h). The last down block resets the counters for
// the next launch unless the error word is set.
// Workspace: h [128][I] bf16 | the down GEMM's split-K partials and arrival
// counters | sync (128 S + 256 bytes): slice counter s at +128 s, done at
// +128 S, error at +128 S + 128 (the last line but one).
// BLOCK: all three weights carry 128 x 128 block scales.
template <int GU_BN, int DN_BN, int WGM, int WGN, int GU_NSA, int GU_NSB, int DN_NSA, int DN_NSB,
          bool BLOCK = false>
struct GatedMlpGemm {
  using GU = Tile<GU_BN, WGM, WGN, GU_NSA, GU_NSB>;
  using DN = Tile<DN_BN, WGM, WGN, DN_NSA, DN_NSB>;
  static constexpr int kSmem = GU::kSmem > DN::kSmem ? GU::kSmem : DN::kSmem;
  LF_DEVICE static void run(const int32_t *counts, const uint16_t *x, const uint8_t *wg,
                            const uint8_t *wu, const uint8_t *wd, uint16_t *y, uint8_t *ws) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmem];
    __shared__ phase::Flag flag;
    constexpr uint32_t kScale = BLOCK ? kScaleBlock128 : kScalePerChannel;
    if (!dense_regions_ok<2, kScale>(wg, wu, wu) || !dense_regions_ok<0, kScale>(wd, wd, wd)) return;
    const int H = static_cast<int>(header_of(wg).columns), I = static_cast<int>(header_of(wg).rows);
    if (static_cast<int>(header_of(wd).columns) != I || static_cast<int>(header_of(wd).rows) != H) return;
    const int g1 = I / (GU_BN / 2);
    const int g2 = static_cast<int>(gridDim.x) - g1;
    const int dn_blocks_n = H / DN_BN;
    if (g1 < 1 || dn_blocks_n < 1 || g2 < dn_blocks_n || g2 % dn_blocks_n != 0) return;
    const int S = g2 / dn_blocks_n;
    uint16_t *h = reinterpret_cast<uint16_t *>(ws);
    uint8_t *ws_down = ws + align256(128ull * I * 2);
    // (the down GEMM's own workspace size: 256 bytes, unused, without a split)
    const uint64_t down_bytes =
        S == 1 ? 256
               : align256(static_cast<uint64_t>(S) * dn_blocks_n * DN::kWaves * DN::kFM * DN::kFN * 1024) +
                     align256(static_cast<uint64_t>(dn_blocks_n) * 4);
    int *sync = reinterpret_cast<int *>(ws_down + down_bytes);
    int *done = sync + phase::kLineInts * S;
    int *error = done + phase::kLineInts;
    const int KT = I >> 7;
    auto slice_of = [&](int kt) {  // the down K-slice [KT s / S, KT (s + 1) / S) holding k-tile kt
      int sl = 0;
      while (sl + 1 < S && (KT * (sl + 1)) / S <= kt) ++sl;
      return sl;
    };
    const int b = static_cast<int>(blockIdx.x);
    if (b < g1) {
      w8a16_gemm_kernel<GU_BN, WGM, WGN, GU_NSA, GU_NSB, 2, true, NoWait, BLOCK>(smem, counts, x, wg, wu, wu,
                                                                                 h, ws_down, b, g1);
      phase::signal(sync + phase::kLineInts * slice_of(b * (GU_BN / 2) / 128));
      return;
    }
    const auto gate = [&](int sl) {
      const int target = (KT * (sl + 1) / S - KT * sl / S) * (128 / (GU_BN / 2));
      return phase::wait_for(sync + phase::kLineInts * sl, target, error, flag);
    };
    w8a16_gemm_kernel<DN_BN, WGM, WGN, DN_NSA, DN_NSB, 0, false, decltype(gate), BLOCK>(
        smem, counts, h, wd, wd, wd, y, ws_down, b - g1, g2, gate);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int before = __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == g2 - 1 && phase::load_agent(error) == 0) {
        for (int sl = 0; sl < S; ++sl) phase::store_agent(sync + phase::kLineInts * sl, 0);
        phase::store_agent(done, 0);
      }
    }
  }
};

}  // namespace w16g

extern "C" {

// Symbols: lf_fp8_w8a16_{op}_m128_n{BN}; the launch geometry picks BN and the
// K split S (grid = column blocks x S; blocks of 64 WGM WGN threads).
#define LF_W16_GEMM_ENTRIES(BN, WGM, WGN, NSA, NSB)                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_dense_m128_n##BN(               \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) {     \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[w16g::Tile<BN, WGM, WGN, NSA, NSB>::kSmem]; \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 0>(smem, counts, x, w, w, w, y, ws);          \
  }                                                                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_qkv_m128_n##BN(                 \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,            \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                             \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[w16g::Tile<BN, WGM, WGN, NSA, NSB>::kSmem]; \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 1>(smem, counts, x, wq, wk, wv, y, ws);       \
  }                                                                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_gate_up_m128_n##BN(             \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      uint16_t *h, uint8_t *ws) {                                                                \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[w16g::Tile<BN, WGM, WGN, NSA, NSB>::kSmem]; \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 2>(smem, counts, x, wg, wu, wu, h, ws);       \
  }

LF_W16_GEMM_ENTRIES(64, 4, 2, 3, 4)
LF_W16_GEMM_ENTRIES(128, 2, 4, 2, 4)

// The same over weights with 128 x 128 block scales:
// lf_fp8_w8a16_{op}_b128_m128_n{BN}.
#define LF_W16_GEMM_B128_ENTRIES(BN, WGM, WGN, NSA, NSB)                                         \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_dense_b128_m128_n##BN(          \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) {     \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[w16g::Tile<BN, WGM, WGN, NSA, NSB>::kSmem]; \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 0, false, NoWait, true>(smem, counts, x, w, w, w, y, ws); \
  }                                                                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_qkv_b128_m128_n##BN(            \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,            \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                             \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[w16g::Tile<BN, WGM, WGN, NSA, NSB>::kSmem]; \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 1, false, NoWait, true>(smem, counts, x, wq, wk, wv, y, \
                                                                            ws);                 \
  }                                                                                              \
  __global__ __launch_bounds__(64 * WGM * WGN) void lf_fp8_w8a16_gate_up_b128_m128_n##BN(        \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      uint16_t *h, uint8_t *ws) {                                                                \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[w16g::Tile<BN, WGM, WGN, NSA, NSB>::kSmem]; \
    w16g::w8a16_gemm_kernel<BN, WGM, WGN, NSA, NSB, 2, false, NoWait, true>(smem, counts, x, wg, wu, wu, h, \
                                                                            ws);                 \
  }

LF_W16_GEMM_B128_ENTRIES(64, 4, 2, 3, 4)
LF_W16_GEMM_B128_ENTRIES(128, 2, 4, 2, 4)

// One-launch GatedMlp for profiles of 65..128 rows, any H and I the forms
// divide: gate/up on the n128 tiles (one K-slice), down on n128 or n64 (the
// tile and split its own launch would take), operands (counts, x, wg, wu,
// wd, y, ws).
#define LF_W16_GEMM_GATED_MLP(DN_BN, DN_NSA, DN_NSB, WGM, WGN)                                   \
  __global__ __launch_bounds__(512) void lf_fp8_w8a16_gated_mlp_m128_n128_n##DN_BN(               \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      const uint8_t *wd, uint16_t *y, uint8_t *ws) {                                             \
    w16g::GatedMlpGemm<128, DN_BN, WGM, WGN, 2, 4, DN_NSA, DN_NSB>::run(counts, x, wg, wu, wd, y, ws); \
  }

LF_W16_GEMM_GATED_MLP(128, 2, 4, 2, 4)
LF_W16_GEMM_GATED_MLP(64, 3, 4, 4, 2)

// The same over weights with 128 x 128 block scales.
#define LF_W16_GEMM_GATED_MLP_B128(DN_BN, DN_NSA, DN_NSB, WGM, WGN)                              \
  __global__ __launch_bounds__(512) void lf_fp8_w8a16_gated_mlp_b128_m128_n128_n##DN_BN(          \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      const uint8_t *wd, uint16_t *y, uint8_t *ws) {                                             \
    w16g::GatedMlpGemm<128, DN_BN, WGM, WGN, 2, 4, DN_NSA, DN_NSB, true>::run(counts, x, wg, wu, wd, y, ws); \
  }

LF_W16_GEMM_GATED_MLP_B128(128, 2, 4, 2, 4)
LF_W16_GEMM_GATED_MLP_B128(64, 3, 4, 4, 2)

}  // extern "C"
