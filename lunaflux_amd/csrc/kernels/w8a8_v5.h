// w8a8_v5.h - e4m3 x e4m3 MFMA main loop for 256-row tiles on four waves:
// one wave per SIMD, each owning 128 rows x BN / 2 columns of
// v_mfma_scale_f32_16x16x128_f8f6f4 (unit scales, accumulators in the AGPR
// file), LDS stages of 128-deep k-tiles filled by global_load_lds_dwordx4:
// 256 x 256 tiles on two 64 KiB stages (Tile), 256 x 128 tiles on three
// 48 KiB stages (TileN128).
//
// Stage layout, load plan and fragment reads are those of w8a8_v3.h's loop
// (A rows with the chunk swizzle that reads conflict-free, B as verbatim
// 2 KiB weight tiles), on w8a8v3 tiles of 2 x 2 waves. The load addresses
// are held as wave-uniform 64-bit bases in scalar registers plus 32-bit
// per-lane offsets (Plan): the A rows of the tile from one base (tile row
// offset times K plus the chunk: K < 2^24 keeps it in 32 bits), each B
// half-tile's base with the lane's 16 bytes as the one shared offset. This
// takes 9 vector registers where 64-bit per-lane addresses took 32.
//
// Against the 8-wave half-step loop (w8a8_v4.h) a wave keeps its 128 x 128
// block of outputs (256 x 256 tiles), so a k-tile reads 64 KiB of fragments
// from LDS per CU instead of 96 KiB (8 A and 8 B fragments of 2 KiB per
// wave, 64 MFMAs each of 32 cycles). With one wave per SIMD nothing else
// covers a stall of the matrix pipe, so the order of one k-tile (8 rows i of
// BN / 32 MFMAs (i, j)) is fixed by hand (sched_barrier):
//   rows 0..P read A fragments 2..7 of stage kt (each at least a row before
//     its use; fragments 0 and 1 and all B fragments were read at the end of
//     the previous k-tile);
//   after row P (barrier_row) the wave has read everything it needs from
//     stage kt: it waits for its own loads of stage kt + 1 (the later stages'
//     loads may stay in flight) and joins the block barrier, after which
//     stage kt + 1 is complete in LDS and no wave reads stage kt's slot any
//     more;
//   the loads of stage kt + NS (NS stages) into that slot are spread evenly
//     over the MFMAs of the remaining rows (one per two MFMAs on 256 x 256):
//     a CU's 64 load instructions of a 256 x 256 k-tile (64 KiB) take the
//     vector memory path about as long as 32 MFMAs take the matrix pipe, and
//     a lone wave that issues them faster stalls at the issue of the next
//     one;
//   row 7: MFMA (7, j) is followed by the read of stage kt + 1's B fragment
//     j (it was the last reader of those registers), and A fragments 0 and
//     1 of stage kt + 1 are read around it.
// On two stages the loads of a stage have the rows from their issue to the
// next k-tile's barrier to land. 256 x 256, barrier after row 5 with the
// loads one per MFMA in rows 6-7, after row 4, 3 and 2, measured on MI355X
// at M = 8192 (K 4096 / 14336 / 4096 x 28672): 114.1 / 111.7 / 108.4 / 108.6
// us for o, 365 / 351 / 340 / 338 us for down, 731 / 719 / 716 / 722 us for
// gate/up.
// SWAP: the weight fragment is the MFMA's first operand, so each 16 x 16
// accumulator holds the transposed block: lane l keeps tile row 16 i + l % 16
// and columns 16 j + 4 (l / 16) + q, q = 0..3 (acc_row / acc_col), which the
// epilogue stores as one 8-byte LDS write per accumulator.
#pragma once

#include <type_traits>

#include "w8a8_v3.h"

namespace w8a8v5 {

using Tile = w8a8v3::Tile<256, 256, 2, 2, 2>;
// 256 x 128 tiles (128 x 64 wave tiles), three 48 KiB stages.
using TileN128 = w8a8v3::Tile<256, 128, 3, 2, 2>;

// Row after which a k-tile waits for the next stage and joins the barrier:
// 3 on two stages (the loads of a stage have one k-tile to land), 1 on
// three (they have two; the earlier barrier spreads them over more rows).
// Measured at M = 1024 / 2048 on 256 x 128 tiles, rows 1 / 2 / 3 / 4: o 35.3
// / 35.4 / 35.4 / 35.8 us and down 108.7 / 109.2 / 108.5 / 109.3 us at M =
// 2048, QKV 34.0 / 34.7 / 34.8 / 35.3 us and down 93.9 / 94.5 / 95.4 / 97.3
// us at M = 1024.
// Load plan: A instruction q of this wave at k-tile kt fetches a_base +
// kt * 128 + a_off[q]; B instruction q fetches b_base[q] + kt * kTileBytes +
// b_lane.
template <class T>
struct Plan {
  const uint8_t *a_base;
  uint32_t a_off[T::kAIns];
  const uint8_t *b_base[T::kBIns];
  uint32_t b_lane;
};


template <class T>
constexpr int barrier_row() {
  return T::kStages == 3 ? 1 : 3;
}

template <class T, bool SWAP, int P = barrier_row<T>()>
__device__ __forceinline__ void mainloop(const Plan<T> &plan, int KT, uint8_t *smem,
                                         f32x4 (&acc)[T::kFM][T::kFN]) {
  constexpr int NS = T::kStages, FM = T::kFM, FN = T::kFN;
  static_assert((NS == 2 || NS == 3) && FM == 8 && T::kWaves == 4, "4-wave 256-row tile");
  static_assert(T::kAIns == 8, "8 A loads per wave and stage");
  constexpr int R = FM - 1 - P;  // rows after the barrier
  static_assert(P >= 1 && P <= 5, "A fragments 2..7 are read in rows 0..P");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;
  const int g = lane >> 4, r = lane & 15;
  const uint32_t smem_base = __builtin_amdgcn_readfirstlane(w8a8v3::lds_offset_of(smem));
  // Load q of stage kt: q < 8 are this wave's A instructions, the rest its B
  // instructions (w8a8v3 plan order).
  auto dma = [&](int kt, int q) {
    const uint32_t a = smem_base + (kt % NS) * T::kStage;
    if (q < T::kAIns) {
      w8a8v3::dma16(plan.a_base + kt * 128, plan.a_off[q], a + (wave * T::kAIns + q) * 1024);
    } else {
      w8a8v3::dma16(plan.b_base[q - T::kAIns] + kt * kTileBytes, plan.b_lane,
                    a + T::kABytes + w8a8v3::b_load_half<T>(wave, q - T::kAIns) * 1024);
    }
  };
  auto stage = [&](int kt) -> const uint8_t * { return smem + (kt % NS) * T::kStage; };
  // Fragment rows of one 16-row block keep the same swizzle 16 rows further
  // (it depends on row & 7 only), so A fragment i is a_off + 2048 i.
  const int row0 = wm * T::kWaveM + r;
  const int a_off0 = w8a8v3::a_chunk_offset(row0, 2 * g);
  const int a_off1 = w8a8v3::a_chunk_offset(row0, 2 * g + 1);
  const int b_off = T::kABytes + wn * FN * kTileBytes + lane * 16;
  w8a8::Frag8 bf[FN], af[FM];
  auto read_a = [&](int i, const uint8_t *st) {
    af[i].h[0] = *reinterpret_cast<const uint4 *>(st + a_off0 + 2048 * i);
    af[i].h[1] = *reinterpret_cast<const uint4 *>(st + a_off1 + 2048 * i);
  };
  auto read_b = [&](int j, const uint8_t *st) {
    bf[j].h[0] = *reinterpret_cast<const uint4 *>(st + b_off + kTileBytes * j);
    bf[j].h[1] = *reinterpret_cast<const uint4 *>(st + b_off + kTileBytes * j + 1024);
  };
  auto mfma = [&](int i, int j) {
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        SWAP ? bf[j].v : af[i].v, SWAP ? af[i].v : bf[j].v, acc[i][j], 0, 0, 0, 127, 0, 127);
  };
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: stages 0 .. NS - 1 in flight, wait for stage 0 (loads complete
  // in issue order), read its B fragments and A fragments 0 and 1.
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (s < KT) {
#pragma unroll
      for (int q = 0; q < T::kIns; ++q) dma(s, q);
    }
  }
  if (NS == 3 && KT >= 3) {
    w8a8v3::wait_vmcnt<(NS - 1) * T::kIns>();
  } else if (KT >= 2) {
    w8a8v3::wait_vmcnt<T::kIns>();
  } else {
    w8a8v3::wait_vmcnt<0>();
  }
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int j = 0; j < FN; ++j) read_b(j, stage(0));
  read_a(0, stage(0));
  read_a(1, stage(0));

  // NEXT: stage kt + 1 exists (wait, barrier, its fragment reads); ISSUE:
  // stage kt + NS exists (its loads go to stage kt's slot); LATER: stages
  // issued after kt + 1 whose loads may still be in flight at the barrier
  // (0 or, with three stages, 1). Compile-time, so the k-tile body has no
  // branches.
  auto step = [&](auto next_tag, auto issue_tag, auto later_tag, int kt) {
    constexpr bool kNext = decltype(next_tag)::value, kIssue = decltype(issue_tag)::value;
    constexpr int kLater = decltype(later_tag)::value;
    const uint8_t *st = stage(kt);
    const uint8_t *nx = stage(kt + 1);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if (i <= P) {
        // A fragment f (2..7) is read in row (f - 2)(P + 1) / 6 <= f - 2.
#pragma unroll
        for (int f = 2; f < FM; ++f) {
          if ((f - 2) * (P + 1) / 6 == i) read_a(f, st);
        }
      }
      if (kNext && i == FM - 1) read_a(0, nx);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        mfma(i, j);
        __builtin_amdgcn_sched_barrier(0);
        if (kIssue && i > P) {
          // load q goes after MFMA slot q FN R / kIns of the FN R after the
          // barrier
          const int s = (i - P - 1) * FN + j;
#pragma unroll
          for (int q = 0; q < T::kIns; ++q) {
            if ((q * FN * R) / T::kIns == s) dma(kt + NS, q);
          }
        }
        if (kNext && i == FM - 1) read_b(j, nx);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kNext && i == P) {
        w8a8v3::wait_vmcnt<kLater * T::kIns>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (kNext) read_a(1, nx);
  };
  using Yes = std::true_type;
  using No = std::false_type;
  using L0 = std::integral_constant<int, 0>;
  using LN = std::integral_constant<int, NS - 2>;
  int kt = 0;
  for (; kt + NS < KT; ++kt) step(Yes{}, Yes{}, LN{}, kt);
  // kt + NS >= KT: nothing left to issue; the stages after kt + 1 still in
  // flight number KT - 2 - kt (at most NS - 2).
  if (NS == 3 && kt + 2 < KT) {
    step(Yes{}, No{}, LN{}, kt);
    ++kt;
  }
  if (kt + 1 < KT) {
    step(Yes{}, No{}, L0{}, kt);
    ++kt;
  }
  step(No{}, No{}, L0{}, kt);
}

// Wave-tile row and column of element q of accumulator (i, j) of lane `lane`
// in the SWAP layout.
LF_DEVICE int acc_row(int i, int lane) { return 16 * i + (lane & 15); }
LF_DEVICE int acc_col(int j, int lane, int q) { return 16 * j + 4 * (lane >> 4) + q; }

}  // namespace w8a8v5
