// w8a8_v3.h - e4m3 x e4m3 MFMA main loop with direct global-to-LDS loads.
//
// Block tile BM x BN x 128 (K per step), WGM x WGN waves (64 WGM WGN
// threads), wave tile (BM/WGM) x (BN/WGN) of v_mfma_scale_f32_16x16x128_f8f6f4
// (unit scales).
// Operands move global -> LDS with global_load_lds_dwordx4 (no register
// staging): each wave instruction writes 1 KiB of LDS contiguously, lane l
// at +16 l. NS LDS stages form a ring and the loads of k-step kt + NS - 1 are
// issued while k-step kt computes, so L2/HBM latency is covered without
// occupancy. Stage layout:
//   A: BM rows x 128 bytes; LDS row r holds the row's 16-byte chunk c at
//      physical chunk c ^ (((r & 3) << 1) | ((r >> 2) & 1)). A fragment read
//      gives 16 lanes 16 consecutive rows at one logical chunk; measured on
//      gfx950 (ds_read_b128, 8 waves per CU) this swizzle reads at the
//      contiguous rate, 256 B/clk per CU, where c ^ ((r >> 1) & 7) (row
//      pairs spread over the chunk positions) ran at 2/3 of it. The swizzle
//      is applied on the global side: lane l of a load instruction writes LDS
//      row r = 8 (instr) + l / 8, physical chunk l % 8, so it fetches logical
//      chunk (l % 8) ^ (((r & 3) << 1) | ((r >> 2) & 1)).
//   B: BN/16 pre-swizzled 16 x 128 weight tiles copied verbatim, 2 KiB each.
//
// The caller provides, per lane, the global row base of each A row it loads
// (gathered rows are fine) and the global tile base of each B half-tile.
#pragma once

#include "w8a8_core.h"

namespace w8a8v3 {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

template <int BM, int BN, int NS, int WGM = 2, int WGN = 2>
struct Tile {
  static constexpr int kWaves = WGM * WGN, kThreads = 64 * kWaves;
  static constexpr int kWaveM = BM / WGM, kWaveN = BN / WGN;
  static constexpr int kFM = kWaveM / 16, kFN = kWaveN / 16;
  static constexpr int kABytes = BM * 128, kBBytes = BN * 128;
  static constexpr int kStage = kABytes + kBBytes;
  static constexpr int kSmem = NS * kStage;
  static constexpr int kStages = NS, kWgm = WGM, kWgn = WGN;
  // 1 KiB load instructions per wave and stage
  static constexpr int kAIns = BM / (8 * kWaves), kBIns = BN / (8 * kWaves);
  static constexpr int kIns = kAIns + kBIns;
  static_assert(kSmem <= 160 * 1024, "LDS budget");
  static_assert(kAIns * 8 * kWaves == BM && kBIns * 8 * kWaves == BN, "load split");
  static_assert(kWaveM % 16 == 0 && kWaveN % 32 == 0, "wave tile");
};

// Tile row loaded by lane `lane` of this wave's A instruction q.
template <class T>
LF_DEVICE int a_load_row(int wave, int q, int lane) {
  return 8 * (wave * T::kAIns + q) + (lane >> 3);
}
// Physical chunk of logical 16-byte chunk `chunk` of tile row `row`, and the
// byte offset of that chunk in a stage.
LF_DEVICE int a_phys_chunk(int row, int chunk) { return chunk ^ (((row & 3) << 1) | ((row >> 2) & 1)); }
LF_DEVICE int a_chunk_offset(int row, int chunk) { return row * 128 + (a_phys_chunk(row, chunk) << 4); }
// Logical 16-byte chunk of that row this lane fetches.
LF_DEVICE int a_load_chunk(int row, int lane) { return a_phys_chunk(row, lane & 7); }
// B half-tile (2 per 16-column slot) of this wave's B instruction q.
template <class T>
LF_DEVICE int b_load_half(int wave, int q) { return wave * T::kBIns + q; }

template <class T>
struct Plan {
  // a[q]: global address of this lane's 16 bytes of A instruction q at k = 0
  // (row base + logical chunk * 16); b[q]: global address of its 16 bytes of
  // B instruction q at k-tile 0 (strip base + half * 1024 + lane * 16).
  const uint8_t *a[T::kAIns];
  const uint8_t *b[T::kBIns];
};

template <int N>
LF_DEVICE void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One global_load_lds_dwordx4: every lane fetches 16 bytes from its global
// address and the wave writes them to LDS at lds_offset + 16 * lane. Issued
// as inline assembly so the compiler does not model the LDS write: it would
// otherwise make every LDS read wait for all outstanding loads (including
// the prefetch of later stages). The main loop orders these writes against
// the LDS reads itself (s_waitcnt vmcnt + block barrier). M0 carries the
// LDS offset, which must be wave-uniform (the compiler cannot prove that of
// values derived from threadIdx.x, hence the readfirstlane); no other code in
// these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is listed as clobbered on purpose
LF_DEVICE void dma16(const uint8_t *src, uint32_t lds_offset) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_offset))
               : "memory", "m0");
}
// A pointer every lane of the wave holds, moved to scalar registers.
LF_DEVICE const uint8_t *uniform_ptr(const uint8_t *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The same load with a wave-uniform base in scalar registers and a 32-bit
// lane offset (address base + offset): the loops keep one base per
// instruction group and a 32-bit register per lane instead of a 64-bit
// address per lane and instruction.
LF_DEVICE void dma16(const uint8_t *base, uint32_t offset, uint32_t lds_offset) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(offset), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds_offset))
               : "memory", "m0");
}
// The same for 4 bytes per lane: lane l's dword lands at lds_offset + 4 l.
LF_DEVICE void dma4(const uint8_t *base, uint32_t offset, uint32_t lds_offset) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(offset), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds_offset))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte offset of a pointer into a __shared__ array (an address-space
// conversion, which only a C-style cast expresses).
LF_DEVICE uint32_t lds_offset_of(const uint8_t *p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)p));
}

// Folds of the per-k-tile products into the accumulators. NoFold: the MFMAs
// accumulate into acc directly (one scale per row and per column, applied
// in the epilogue). A folding functor (kActive = true) receives each
// k-tile's products in fresh registers instead and adds them to acc with
// its own factors (block scales that change with k).
struct NoFold {
  static constexpr bool kActive = false;
  template <class A>
  LF_DEVICE void operator()(int, const A &, A &, int) const {}
};

// Side loads: Side::kIns more LDS-direct loads per wave and k-step, issued
// right after the stage's own loads (side.issue(kt, slot), slot = kt % NS)
// and waited for with them, so what they bring is in LDS when fold(kt)
// runs and stays there until the k-step's slot is reused NS steps later.
// NoSide: none.
struct NoSide {
  static constexpr int kIns = 0;
  LF_DEVICE void issue(int, int) const {}
};

// SKIP: live_fm is how many of this wave's kFM 16-row fragments hold a live
// row (wave-uniform); a wave with none skips its A reads, MFMAs and folds
// (its accumulators are never stored). Skipping single fragments cost the
// block-scaled kernel an occupancy step in registers, so the skip is per
// wave. Only the grouped GEMMs, whose expert tiles are often partly past the
// expert's last row, use it.
template <class T, class Fold = NoFold, bool SKIP = false, class Side = NoSide>
__device__ __forceinline__ void mainloop(const Plan<T> &plan, int KT, uint8_t *smem,
                         f32x4 (&acc)[T::kFM][T::kFN], const Fold &fold = Fold{},
                         int live_fm = T::kFM, const Side &side = Side{}) {
  const int live = __builtin_amdgcn_readfirstlane(live_fm);
  constexpr int NS = T::kStages;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;
  const int g = lane >> 4, r = lane & 15;

  const uint32_t smem_base = __builtin_amdgcn_readfirstlane(lds_offset_of(smem));
  auto issue = [&](int kt) {
    const uint32_t a = smem_base + (kt % NS) * T::kStage;
    const uint32_t b = a + T::kABytes;
#pragma unroll
    for (int q = 0; q < T::kAIns; ++q) {
      dma16(plan.a[q] + kt * 128, a + (wave * T::kAIns + q) * 1024);
    }
#pragma unroll
    for (int q = 0; q < T::kBIns; ++q) {
      dma16(plan.b[q] + kt * kTileBytes, b + b_load_half<T>(wave, q) * 1024);
    }
    side.issue(kt, kt % NS);
  };

#pragma unroll
  for (int i = 0; i < T::kFM; ++i)
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < NS - 1; ++s) {
    if (s < KT) issue(s);
  }
  for (int kt = 0; kt < KT; ++kt) {
    // Stage kt has landed once at most the loads of the later in-flight
    // stages are outstanding (completions are counted in issue order).
    const int later = KT - 1 - kt < NS - 2 ? KT - 1 - kt : NS - 2;
    if (later >= NS - 2) {
      wait_vmcnt<(NS - 2) * (T::kIns + Side::kIns)>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();  // every wave's part of stage kt is in LDS, and stage
                      // kt - 1 (reused below) is no longer being read
    if (kt + NS - 1 < KT) issue(kt + NS - 1);
    const uint8_t *a = smem + (kt % NS) * T::kStage;
    const uint8_t *b = a + T::kABytes;
    w8a8::Frag8 bf[T::kFN];
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) {
      const uint8_t *tile = b + (wn * T::kFN + j) * kTileBytes;
      bf[j].h[0] = *reinterpret_cast<const uint4 *>(tile + lane * 16);
      bf[j].h[1] = *reinterpret_cast<const uint4 *>(tile + 1024 + lane * 16);
    }
    if (SKIP && live == 0) continue;  // wave-uniform; stage bookkeeping is above
    f32x4 step[Fold::kActive ? T::kFM : 1][Fold::kActive ? T::kFN : 1];
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
      const int row = wm * T::kWaveM + i * 16 + r;
      w8a8::Frag8 af;
      af.h[0] = *reinterpret_cast<const uint4 *>(a + a_chunk_offset(row, 2 * g));
      af.h[1] = *reinterpret_cast<const uint4 *>(a + a_chunk_offset(row, 2 * g + 1));
#pragma unroll
      for (int j = 0; j < T::kFN; ++j) {
        if constexpr (Fold::kActive) {
          step[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              af.v, bf[j].v, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af.v, bf[j].v, acc[i][j], 0,
                                                                       0, 0, 127, 0, 127);
        }
      }
    }
    if constexpr (Fold::kActive) fold(kt, step, acc, T::kFM);
  }
}

template <class T>
LF_DEVICE int acc_row(int wm, int i, int lane, int rr) {
  return wm * T::kWaveM + i * 16 + (lane >> 4) * 4 + rr;
}

// Block -> output tile order for a 1-D grid over the gx x gy tiles that hold
// live rows (blocks past them return). Workgroups are dispatched to the 8
// XCDs round-robin, so block b runs on XCD b % 8; each XCD is given one
// contiguous range of the tile order, and inside it tiles go down groups of
// `group` row blocks column by column, so the blocks resident on an XCD at
// one time share few A row strips and weight column strips in its L2.
// Returns false for blocks with no tile.
// b: the block's index in the GEMM's part of the grid (blockIdx.x when the
// GEMM is the whole grid; a one-launch operation puts other steps' blocks
// first, in a multiple of 8 so that b % 8 is still the XCD).
// group < 0 (striped order, when gx is a multiple of 8): XCD x takes the
// columns x, x + 8, ... and every XCD walks the same groups of -group row
// blocks in turn (inside a group: column by column, down its rows), so the
// first row blocks are done early across the chip instead of every XCD
// finishing its own rows at the end; a column's row tiles still run on one
// XCD, back to back.
LF_DEVICE bool tile_of_block(int b, int gx, int gy, int group, int &bx, int &by) {
  const int tiles = gx * gy;
  if (b >= tiles) return false;
  if (group < 0 && (gx & 7) == 0) {
    const int g = -group, cx = gx >> 3, xcd = b & 7, local = b >> 3;
    const int first = local / (g * cx) * g;
    const int rows = gy - first < g ? gy - first : g;
    const int in = local - first * cx;
    by = first + in % rows;
    bx = (in / rows) * 8 + xcd;
    return true;
  }
  if (group < 0) group = -group;
  const int xcd = b & 7, local = b >> 3;
  const int base = tiles >> 3, extra = tiles & 7;
  const int t = xcd * base + (xcd < extra ? xcd : extra) + local;
  const int span = group * gx;
  const int first = (t / span) * group;
  const int rows = gy - first < group ? gy - first : group;
  const int in = t % span;
  by = first + in % rows;
  bx = in / rows;
  return true;
}
LF_DEVICE bool tile_of_block(int gx, int gy, int group, int &bx, int &by) {
  return tile_of_block(static_cast<int>(blockIdx.x), gx, gy, group, bx, by);
}

}  // namespace w8a8v3
