// w8a8_v4.h - e4m3 x e4m3 MFMA main loop: direct global-to-LDS loads in
// 64-deep K half-steps, v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales),
// fragments double-buffered in registers.
//
// Block tile BM x BN, WGM x WGN waves, wave tile (BM/WGM) x (BN/WGN) of
// 32 x 32 MFMA blocks. K advances in half-steps of 64: half-step s covers
// half h = s & 1 of k-tile s >> 1, and "half h" is the set of k with
// (k / 16) % 2 == h, i.e. 16-byte chunks h, h+2, h+4, h+6 of a 128-byte
// k-tile row. That set is exactly the h-th 1 KiB half of a packed 16 x 128
// weight tile (lane l of half h holds column l % 16, k = 32 (l / 16) + 16 h
// + 0..15), so the packed weight format needs no change. Any permutation of
// K is valid for a dot product as long as A and B agree, which they do.
//
// LDS stage (NS of them, a ring):
//   A: BM rows x 64 bytes. Row r keeps its 4 chunks (slot j = logical chunk
//      2 j + h) at physical slot j ^ ((r >> 2) & 3). A ds_read_b128 is served
//      16 lanes (256 bytes, all banks) at a time; a fragment read gives them
//      16 consecutive rows at one logical slot: rows 4k..4k+3 fill the four
//      64-byte quarters of a bank window and (r >> 2) & 3 moves the slot, so
//      the 16 lanes of a pass hit 16 distinct 16-byte bank groups.
//   B: BN / 16 tile halves of 1 KiB, copied verbatim.
// MFMA operands (lane l, q = l / 32): A row 32 i + l % 32 and B column
// 32 j + l % 32, each with slots 2q and 2q+1 (32 bytes).
//
// Schedule per half-step s: wait until this wave's loads of stage s + 1 have
// landed, block barrier (stage s + 1 visible everywhere; the slot being
// refilled was last read two half-steps ago), issue the loads of stage
// s + NS - 1, then the MFMAs of stage s interleaved with the LDS reads of
// stage s + 1's fragments into the other register set.
#pragma once

#include <type_traits>

#include "phases.h"
#include "w8a8_v3.h"

namespace w8a8v4 {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int BM, int BN, int NS, int WGM, int WGN>
struct Tile {
  static constexpr int kWaves = WGM * WGN, kThreads = 64 * kWaves;
  static constexpr int kWaveM = BM / WGM, kWaveN = BN / WGN;
  static constexpr int kFM = kWaveM / 32, kFN = kWaveN / 32;
  static constexpr int kABytes = BM * 64, kBBytes = BN * 64;
  static constexpr int kStage = kABytes + kBBytes;
  static constexpr int kSmem = NS * kStage;
  static constexpr int kStages = NS, kWgm = WGM, kWgn = WGN, kBM = BM, kBN = BN;
  // 1 KiB load instructions per wave and half-step: 16 A rows, or one
  // weight tile half, each.
  static constexpr int kAIns = BM / (16 * kWaves), kBIns = BN / (16 * kWaves);
  static constexpr int kIns = kAIns + kBIns;
  static_assert(NS == 4, "the main loop's schedule is written for a 4-stage ring");
  static_assert(kSmem <= 160 * 1024, "LDS budget");
  static_assert(kAIns * 16 * kWaves == BM && kBIns * 16 * kWaves == BN, "load split");
  static_assert(kWaveM % 32 == 0 && kWaveN % 32 == 0, "wave tile");
};

LF_DEVICE int a_phys_slot(int row, int slot) { return slot ^ ((row >> 2) & 3); }

// Tile row written by lane `lane` of this wave's A instruction q, and the
// logical slot it fetches (its physical slot is lane & 3).
template <class T>
LF_DEVICE int a_load_row(int wave, int q, int lane) {
  return 16 * (wave * T::kAIns + q) + (lane >> 2);
}
LF_DEVICE int a_load_slot(int row, int lane) { return a_phys_slot(row, lane & 3); }
// Block-local weight tile loaded by this wave's B instruction q.
template <class T>
LF_DEVICE int b_load_tile(int wave, int q) { return wave * T::kBIns + q; }

// Load plan, wave-uniform bases (scalar registers) plus 32-bit lane offsets:
// A instruction q at k-tile kt, half h fetches a_base + kt * 128 + h * 16 +
// a_off[q] (a_off: the row's offset from a_base + 32 * logical slot); B
// instruction q fetches b_base[q] + kt * kTileBytes + h * 1024 + b_lane
// (b_base: the tile strip; b_lane = 16 * lane).
template <class T>
struct Plan {
  const uint8_t *a_base;
  uint32_t a_off[T::kAIns];
  const uint8_t *b_base[T::kBIns];
  uint32_t b_lane;
};

// Block barrier without the memory fence of __syncthreads (which would make
// the compiler wait for every outstanding LDS read first). The "memory"
// clobber keeps the compiler from moving loads or stores across it; the
// ordering the loop needs is enforced with explicit counter waits.
LF_DEVICE void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// SKIP: live_fm is how many of this wave's kFM 32-row fragments hold a live
// row (wave-uniform); the MFMAs of the others are skipped (their
// accumulators stay zero and are never stored), which frees the matrix pipe
// of a SIMD for its other wave when a tile is partly past the last row. The
// branches cost full tiles a few percent (measured on the dense prefill
// GEMMs, whose only partial tile is the last row tile), so only the grouped
// GEMMs, where partial tiles are common, use this form.
// RESCALE (block-scaled operands): before the first half-step of k-tile kt,
// rescale.begin(kt) loads that k-tile's multipliers and rescale.apply(o, acc)
// multiplies the accumulators of column fragment o right before their first
// MFMA of the k-tile (NoRescale: per-channel scales, nothing to do). The
// loop works on its own copy of the functor.
// a_loads (wave-uniform): whether this wave issues its A loads. A wave loads
// A rows 16 kAIns wave .. + 16 kAIns - 1; when all of them are past the last
// live row the caller passes false and the wave issues only its B loads.
// Every fragment an MFMA reads then still comes from a loading wave,
// provided the caller's live_fm skips each fragment whose rows are all dead
// and the fragments line up with the loaders' row ranges (kAIns = 2: 32 rows
// per loader and per fragment). The rows such a wave would have written keep
// whatever the LDS held; no MFMA reads them. Each wave counts its own loads
// (vmcnt), so the waits use kBIns loads per stage for such a wave.
// SIDE: extra loads of each stage (Side::kIns DMA instructions per wave,
// e.g. a block-scaled operand's per-k-tile scales into an LDS window),
// issued after the stage's own loads, so the waits count them
// (w8a8v3::NoSide: none).
// SWAP: the MFMAs take the weight fragment as their first operand and the
// activation fragment as the second, so each accumulator block holds the
// transposed product: lane l keeps tile row 32 i + l % 32 of fragment i and,
// for element 4 g + q of fragment j, column 32 j + 8 g + 4 (l / 32) + q (one
// row per lane and fragment, runs of 4 consecutive columns; acc_row_t and
// acc_col_t). The sums are the same, element by element.
struct NoRescale {
  LF_DEVICE void begin(int) {}
  template <class A>
  LF_DEVICE void apply(int, A &) {}
};

template <class T, bool SKIP = false, class Rescale = NoRescale, bool SWAP = false,
          class Side = w8a8v3::NoSide>
__device__ __forceinline__ void mainloop(const Plan<T> &plan, int KT, uint8_t *smem,
                         f32x16 (&acc)[T::kFM][T::kFN], int live_fm = T::kFM,
                         Rescale rescale = Rescale{}, bool a_loads = true,
                         const Side &side = Side{}) {
  static_assert(!SKIP || T::kAIns * 16 == 32, "a loader's rows are one 32-row fragment");
  constexpr int NS = T::kStages;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;
  const int q = lane >> 5, c = lane & 31;
  const int S = 2 * KT;
  const bool a_on = !SKIP || __builtin_amdgcn_readfirstlane(static_cast<int>(a_loads)) != 0;

  // Wait until at most N stages of this wave's loads are outstanding.
  auto wait_stages = [&](auto n_tag) {
    constexpr int N = decltype(n_tag)::value;
    if (a_on) {
      w8a8v3::wait_vmcnt<N * (T::kIns + Side::kIns)>();
    } else {
      w8a8v3::wait_vmcnt<N * (T::kBIns + Side::kIns)>();
    }
  };
  const uint32_t smem_base = __builtin_amdgcn_readfirstlane(w8a8v3::lds_offset_of(smem));
  // Load q of stage s: this wave's A instructions first, then its B ones.
  auto issue_one = [&](int s, int q) {
    const int kt = s >> 1, h = s & 1;
    const uint32_t a = smem_base + (s % NS) * T::kStage;
    if (q < T::kAIns) {
      if (a_on) {
        w8a8v3::dma16(plan.a_base + kt * 128 + h * 16, plan.a_off[q], a + (wave * T::kAIns + q) * 1024);
      }
    } else {
      w8a8v3::dma16(plan.b_base[q - T::kAIns] + kt * kTileBytes + h * 1024, plan.b_lane,
                    a + T::kABytes + b_load_tile<T>(wave, q - T::kAIns) * 1024);
    }
  };
  auto issue = [&](int s) {
#pragma unroll
    for (int q = 0; q < T::kIns; ++q) issue_one(s, q);
    side.issue(s, s % NS);
  };

  // LDS byte offsets of this lane's fragment reads inside a stage: A block i
  // at a_off0 / a_off1 (slots 2q, 2q+1) + 2048 i (32 rows further keep the
  // same swizzle: (r + 32) >> 2 & 3 == r >> 2 & 3), B block j at b_off +
  // 2048 j and + 256.
  const int row0 = wm * T::kWaveM + c;
  const int a_off0 = row0 * 64 + (a_phys_slot(row0, 2 * q) << 4);
  const int a_off1 = a_off0 ^ 16;
  const int b_off = T::kABytes + ((wn * T::kWaveN) / 16 + (c >> 4)) * 1024 + (32 * q + (c & 15)) * 16;
  auto read_a = [&](w8a8::Frag8 &f, int i, const uint8_t *st) {
    f.h[0] = *reinterpret_cast<const uint4 *>(st + a_off0 + 2048 * i);
    f.h[1] = *reinterpret_cast<const uint4 *>(st + a_off1 + 2048 * i);
  };
  auto read_b = [&](w8a8::Frag8 &f, int j, const uint8_t *st) {
    f.h[0] = *reinterpret_cast<const uint4 *>(st + b_off + 2048 * j);
    f.h[1] = *reinterpret_cast<const uint4 *>(st + b_off + 2048 * j + 256);
  };
  // The larger operand set ("outer": kOuter fragments) is refilled in place
  // for the next half-step right after its last MFMA; the smaller ("inner")
  // set is double-buffered.
  constexpr bool kOuterN = T::kFN >= T::kFM;
  constexpr int kOuter = kOuterN ? T::kFN : T::kFM, kInner = kOuterN ? T::kFM : T::kFN;
  auto read_outer = [&](w8a8::Frag8 &f, int o, const uint8_t *st) {
    if (kOuterN) read_b(f, o, st); else read_a(f, o, st);
  };
  auto read_inner = [&](w8a8::Frag8 (&f)[kInner], const uint8_t *st) {
#pragma unroll
    for (int n = 0; n < kInner; ++n) {
      if (kOuterN) read_a(f[n], n, st); else read_b(f[n], n, st);
    }
  };
  auto stage_ptr = [&](int s) -> const uint8_t * { return smem + (s % NS) * T::kStage; };

  w8a8::Frag8 outer[kOuter];
  const int live = __builtin_amdgcn_readfirstlane(live_fm);
  auto mfma_group = [&](const w8a8::Frag8(&cur)[kInner], int o) {
#pragma unroll
    for (int n = 0; n < kInner; ++n) {
      // row fragment of this product: n (inner = A) or o (outer = A)
      if (!SKIP || (kOuterN ? n : o) < live) {
        f32x16 &a = kOuterN ? acc[n][o] : acc[o][n];
        const auto &fa = kOuterN ? cur[n].v : outer[o].v;  // activation rows
        const auto &fb = kOuterN ? outer[o].v : cur[n].v;  // weight columns
        a = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(SWAP ? fb : fa, SWAP ? fa : fb, a, 0, 0,
                                                            0, 127, 0, 127);
      }
    }
  };
  // One half-step: compute stage s from outer / cur while stage s + 1's
  // fragments are read into nxt and, behind each outer fragment's last use,
  // into outer. The first MFMA group goes ahead of the wait and the block
  // barrier so the matrix pipe stays busy while waves synchronize.
  // sched_barrier pins this order (the scheduler would otherwise sink each
  // outer read to just before its use and stall on it). WAIT: stages whose
  // loads may stay in flight once stage s + 1 has landed (-1: stage s + 1
  // does not exist: no wait, barrier or reads); ISSUE: whether stage
  // s + NS - 1 exists. Both are compile-time so the body has no branches.
  // EVEN: s is the first half-step of its k-tile (the calls come in pairs).
  auto step = [&](auto wait_tag, auto issue_tag, auto even_tag, w8a8::Frag8(&cur)[kInner],
                  w8a8::Frag8(&nxt)[kInner], int s) {
    constexpr int kWait = decltype(wait_tag)::value;
    constexpr bool kIssue = decltype(issue_tag)::value;
    constexpr bool kEven = decltype(even_tag)::value;
    const uint8_t *st = stage_ptr(s + 1);
    if constexpr (kEven) {
      rescale.begin(s >> 1);
      rescale.apply(0, acc);
    }
    // Loads of stage s + NS - 1 issued after group o: q in [o kIns / kOuter,
    // (o + 1) kIns / kOuter), so they reach the vector memory path spread
    // over the half-step instead of in one run.
    auto issue_after = [&](int o) {
      if constexpr (kIssue) {
#pragma unroll
        for (int q = o * T::kIns / kOuter; q < (o + 1) * T::kIns / kOuter; ++q) issue_one(s + NS - 1, q);
        if (o == kOuter - 1) side.issue(s + NS - 1, (s + NS - 1) % NS);
      }
    };
    mfma_group(cur, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kWait >= 0) {
      wait_stages(std::integral_constant<int, kWait>{});
      block_barrier();
      issue_after(0);
      read_inner(nxt, st);
      read_outer(outer[0], 0, st);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = 1; o < kOuter; ++o) {
      if constexpr (kEven) rescale.apply(o, acc);
      mfma_group(cur, o);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kWait >= 0) {
        read_outer(outer[o], o, st);
        issue_after(o);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using W1 = std::integral_constant<int, 1>;
  using W0 = std::integral_constant<int, 0>;
  using WNone = std::integral_constant<int, -1>;
  using Yes = std::true_type;
  using No = std::false_type;

#pragma unroll
  for (int i = 0; i < T::kFM; ++i)
#pragma unroll
    for (int j = 0; j < T::kFN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Prologue: stages 0 .. min(2, S - 1) in flight; wait for stage 0.
  w8a8::Frag8 f0[kInner], f1[kInner];
  issue(0);
  issue(1);  // S >= 2 always (K is a multiple of 128)
  if (S > 2) {
    issue(2);
    wait_stages(std::integral_constant<int, 2>{});
  } else {
    wait_stages(std::integral_constant<int, 1>{});
  }
  block_barrier();
  read_inner(f0, stage_ptr(0));
#pragma unroll
  for (int o = 0; o < kOuter; ++o) read_outer(outer[o], o, stage_ptr(0));
  // step(s) refills the slot of stage s - 1, whose fragments every wave had
  // read (and consumed) before reaching step(s)'s barrier. In step(s) the
  // stages issued so far end at min(s + 2, S - 1), so stage s + 1 has landed
  // once at most one stage's loads (s + 2) remain.
  int s = 0;
  for (; s + 4 < S; s += 2) {
    step(W1{}, Yes{}, Yes{}, f0, f1, s);
    step(W1{}, Yes{}, No{}, f1, f0, s + 1);
  }
  if (S >= 4) {  // s == S - 4: stage S - 1 is issued last
    step(W1{}, Yes{}, Yes{}, f0, f1, s);
    step(W1{}, No{}, No{}, f1, f0, s + 1);
    s += 2;
  }
  // s == S - 2: nothing left to issue; wait for the last stage.
  step(W0{}, No{}, Yes{}, f0, f1, s);
  step(WNone{}, No{}, No{}, f1, f0, s + 1);
}

// Epilogue staging. A wave's output tile goes through LDS (the stage ring is
// free once every wave has left the main loop) so that global memory gets
// 16-byte row chunks instead of one 2-byte bf16 (or 4-byte fp32) element
// per lane and accumulator register: 8x (4x) fewer store instructions, each
// covering whole 128-byte row segments. The tile is ROWS x COLS elements of
// `Elem`, row pitch COLS + 16 bytes' worth, so the two row groups of one
// accumulator store (rows r and r + 4) fall in different bank halves.
template <typename Elem, int ROWS, int COLS>
struct StageTile {
  static constexpr int kPitch = COLS + 16 / static_cast<int>(sizeof(Elem));  // elements
  static constexpr int kBytes = ROWS * kPitch * static_cast<int>(sizeof(Elem));
  static constexpr int kChunks = ROWS * COLS * static_cast<int>(sizeof(Elem)) / 16;
  static constexpr int kChunksPerRow = COLS * static_cast<int>(sizeof(Elem)) / 16;
  Elem *base;
  LF_DEVICE void put(int row, int col, Elem v) const { base[row * kPitch + col] = v; }
  // Four consecutive 16-bit elements from column col (a multiple of 4): one
  // 8-byte write.
  LF_DEVICE void put4(int row, int col, const uint32_t (&b)[4]) const {
    static_assert(sizeof(Elem) == 2, "four 16-bit elements");
    *reinterpret_cast<uint2 *>(base + row * kPitch + col) = uint2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
  }
  // Writes the staged tile: row `row` goes to row_ptr(row) (null: skipped).
  // THROUGH: the stores write through the XCD's L2 (phases.h), for a tile
  // that blocks of the same launch read.
  template <bool THROUGH = false, class RowPtr>
  LF_DEVICE void flush(int lane, RowPtr row_ptr) const {
#pragma unroll
    for (int q = 0; q < kChunks / 64; ++q) {
      const int idx = q * 64 + lane;
      const int row = idx / kChunksPerRow, chunk = idx % kChunksPerRow;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(
          reinterpret_cast<const uint8_t *>(base + row * kPitch) + chunk * 16);
      Elem *dst = row_ptr(row);
      if (dst != nullptr) {
        uint8_t *p = reinterpret_cast<uint8_t *>(dst) + chunk * 16;
        if constexpr (THROUGH) {
          phase::store16_through(p, v);
        } else {
          *reinterpret_cast<u32x4 *>(p) = v;
        }
      }
    }
  }
};

// All waves have left the main loop (their last fragment reads are done), so
// the stage ring may be overwritten.
LF_DEVICE void epilogue_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Output coordinates of accumulator element e of lane `lane` in 32 x 32
// block (i, j): row inside the wave tile and column inside the wave tile.
template <class T>
LF_DEVICE int acc_row(int i, int lane, int e) {
  return 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
template <class T>
LF_DEVICE int acc_col(int j, int lane) {
  return 32 * j + (lane & 31);
}
// The same with SWAP: the row is the lane's, the columns run in groups of 4.
template <class T>
LF_DEVICE int acc_row_t(int i, int lane) {
  return 32 * i + (lane & 31);
}
template <class T>
LF_DEVICE int acc_col_t(int j, int lane, int e) {
  return 32 * j + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}

}  // namespace w8a8v4
