// w8a16.hip - W8A16 (decode regime): bf16 activations x e4m3 weights.
//
// Work split. Each wave owns one 16-column output tile (for gate/up: the
// gate and the up tile of the same 16 h-columns) and a block of WAVES waves
// owns WAVES adjacent tiles (a "column group") over one K-slice. The grid is
// column groups x S K-slices (S, the split-K factor, comes from the launch
// geometry: gridDim.x = groups * S). Every weight byte is read by exactly one
// wave; the activation slice x[0:M, slice] streams once per block through a
// two-buffer LDS ring (D k-tiles per buffer) shared by its waves, so
// activation traffic is (columns per block) times smaller than with one
// block per tile.
//
// Per wave: weight k-tiles (two coalesced 1 KiB loads each) are kept D deep
// in flight in a register ring, converted to bf16 in registers (exact) and
// fed to 16x16x32 bf16 MFMAs whose A fragments come from the LDS ring. The
// channel scales and the first activation chunk (global_load_lds straight
// into LDS) are requested first, then the weight ring, so no global latency
// sits between the last weight byte and the stores.
//
// Split-K (S > 1): each block writes its fp32 partial tile to the workspace,
// then the last block of the column group to arrive (an atomic counter per
// group; the last block also resets it to 0 for the next launch) sums the S
// partials in slice order 0..S-1 -- a fixed order, so results do not depend
// on which block finishes last -- and runs the epilogue (channel scale, SwiGLU
// for gate/up, bf16 store). No block ever waits for another.
#include "device_common.h"
#include "phases.h"
#include "w8a8_v3.h"

namespace {

union Frag16 {
  uint4 u;
  bf16x8 v;
};

LF_DEVICE int wave_index() { return static_cast<int>(threadIdx.x) >> 6; }

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

// LDS activation ring of a block: two buffers of XC k-tiles of 16*MT rows of
// bf16, k-tile-major (one k-tile = 16*MT rows x 256 bytes); row r keeps its
// 16-byte chunk c at chunk position c ^ chunk_swizzle(r), so the 16 rows of an MFMA
// fragment read fall in distinct banks.
template <int MT, int XC>
struct XRing {
  static constexpr int kRows = 16 * MT;
  static constexpr int kKTileBytes = kRows * 256;
  static constexpr int kBufferBytes = XC * kKTileBytes;
  static constexpr int kBytes = 2 * kBufferBytes;
  static_assert(kBytes <= 128 * 1024, "LDS budget");
};

// s_waitcnt vmcnt(n * PER) for a wave-uniform n in [1, N].
template <int PER, int N>
LF_DEVICE void wait_vm_multiple(int n) {
  if constexpr (N <= 1) {
    w8a8v3::wait_vmcnt<PER>();
  } else {
    if (n >= N) {
      w8a8v3::wait_vmcnt<N * PER>();
    } else {
      wait_vm_multiple<PER, N - 1>(n);
    }
  }
}

// Epilogue of the column-group forms. Lane element (mt, rr) of acc is output
// row mt*16 + 4g + rr of column out_tile*16 + r (16x16 MFMA accumulator
// layout). S == 1: scale (+ SwiGLU) and store. S > 1 (split-K): the
// workspace holds, per slice, one fp32 accumulator fragment (4 values per
// lane: rows 4g..4g+3 of a 16-row tile) for each (tile, weight, row tile),
// fragment index ((s * tiles + out_tile) * NW + i) * MT + mt, then one
// arrival counter per column group. Row groups wholly past M are neither
// stored nor loaded. The last block of a group to arrive sums the S
// fragments in slice order 0..S-1 (its own from registers) and stores; it
// also resets the group's counter for the next launch.
//
// Partials travel through the device-coherent level without any cache
// maintenance: agent-scope atomic stores and loads write through / bypass
// the per-XCD L2, and this wave's stores are complete (s_waitcnt vmcnt(0))
// before the block's arrival is counted. (A device-scope fence would write
// back and invalidate the whole L2 of the XCD, once per block.)
// Fragment layout: 256 floats, element e of lane l at e * 64 + l, so each
// store or load instruction covers 256 contiguous bytes.
// COHERENT: the outputs are written with agent-scope stores, which write
// through the XCD's L2, so blocks of the same launch on other XCDs can read
// them once the writer's stores have completed.
template <int MT, int NW, int MODE, bool COHERENT = false>
LF_DEVICE void group_epilogue(const f32x4 (&acc)[MT][NW], const float (&sc)[NW], int M, int S,
                              int s, int cg, int tiles, int out_tile, bool active, int ld,
                              uint16_t *y, uint8_t *ws, int &last_block) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, r = lane & 15;
  const int col = out_tile * 16 + r;
  auto finish = [&](int m, const float (&v)[NW]) {
    const float out = MODE == 2 ? silu_mul(v[0] * sc[0], v[NW - 1] * sc[NW - 1]) : v[0] * sc[0];
    const uint16_t bits = static_cast<uint16_t>(f32_to_bf16(out));
    if constexpr (COHERENT) {
      __hip_atomic_store(y + static_cast<uint64_t>(m) * ld + col, bits, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      y[static_cast<uint64_t>(m) * ld + col] = bits;
    }
  };
  if (S == 1) {
    if (!active) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int m = mt * 16 + 4 * g + rr;
        if (m < M) {
          float v[NW];
#pragma unroll
          for (int i = 0; i < NW; ++i) v[i] = acc[mt][i][rr];
          finish(m, v);
        }
      }
    return;
  }

  float *part = reinterpret_cast<float *>(ws);
  int *arrivals = reinterpret_cast<int *>(
      ws + align256(static_cast<uint64_t>(S) * tiles * NW * MT * 256 * sizeof(float)));
  auto frag_at = [&](int slice, int i, int mt) -> float * {
    return part + ((static_cast<uint64_t>(slice) * tiles + out_tile) * NW * MT + i * MT + mt) * 256 + lane;
  };
  if (active) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt * 16 + 4 * g < M) {
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          float *p = frag_at(s, i, mt);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            __hip_atomic_store(p + 64 * e, acc[mt][i][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before =
        __hip_atomic_fetch_add(arrivals + cg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before == S - 1;
    // Every block of the group has arrived: reset for the next launch.
    if (last) __hip_atomic_store(arrivals + cg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_block = last ? 1 : 0;
  }
  __syncthreads();
  if (last_block == 0 || !active) return;
  // Sum the S partial fragments in slice order (this block's own from its
  // registers). Loads of kBatch slices are issued before any is added.
  constexpr int kBatch = 4;
  f32x4 sum[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) sum[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += kBatch) {
    f32x4 v[kBatch][MT][NW];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int slice = s0 + b;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          if (slice < S && slice != s && mt * 16 + 4 * g < M) {
            const float *p = frag_at(slice, i, mt);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[b][mt][i][e] = __hip_atomic_load(p + 64 * e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
          } else {
            v[b][mt][i] = acc[mt][i];
          }
        }
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (s0 + b < S) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < NW; ++i) sum[mt][i] += v[b][mt][i];
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int m = mt * 16 + 4 * g + rr;
      if (m < M) {
        float v[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) v[i] = sum[mt][i][rr];
        finish(m, v);
      }
    }
}

// Block-scaled weights (BLOCK): k-tiles of one slice whose 128 x 128 block
// scales a block keeps in LDS (the geometry splits K so that a slice has at
// most this many).
constexpr int kW16BlockSliceKT = 128;

// MODE 0: dense, 1: qkv (three weights, packed Q|K|V output), 2: gate/up.
// D: weight k-tiles in flight per wave; XC: k-tiles per activation chunk
// (D a multiple of XC).
// BLOCK: the weights carry 128 x 128 block scales (s[N/128][K/128]) instead
// of channel scales. A wave's 16 columns lie in one 128-row block, so each
// k-tile has one scale per weight: the k-tile's four MFMAs accumulate into
// a fresh fragment, which is then multiplied by that scale and added to the
// running sum (y = sum_kt s[nb][kt] sum_{k in kt} x_k q_k, fp32); the
// epilogue applies no channel scale. The slice's scales are staged in LDS
// before the main loop.
template <int WAVES, int MT, int MODE, int D, int XC, bool BLOCK = false>
__device__ void w8a16_kernel(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                             const uint8_t *w1, const uint8_t *w2, uint16_t *y, uint8_t *ws) {
  constexpr int NW = MODE == 2 ? 2 : 1;
  static_assert(D % XC == 0, "a weight ring round covers whole activation chunks");
  using X = XRing<MT, XC>;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[X::kBytes];
  __shared__ int last_block;
  __shared__ float bscale[BLOCK ? WAVES * NW * kW16BlockSliceKT : 1];

  const WeightHeader &h0 = header_of(w0);
  if (!dense_regions_ok<MODE, BLOCK ? kScaleBlock128 : kScalePerChannel>(w0, w1, w2)) return;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = MODE == 1 ? static_cast<int>(h0.rows + header_of(w1).rows + header_of(w2).rows)
                           : static_cast<int>(h0.rows);
  const int tiles = ld >> 4;
  const int groups = (tiles + WAVES - 1) / WAVES;
  const int S = static_cast<int>(gridDim.x) / groups;
  if (S < 1) return;  // the geometry rules this out
  const int cg = static_cast<int>(blockIdx.x) / S;
  const int s = static_cast<int>(blockIdx.x) - cg * S;
  const int kt0 = (KT * s) / S, kt1 = (KT * (s + 1)) / S;
  const int nkt = kt1 - kt0;
  if (cg >= groups || nkt < 1 || (BLOCK && nkt > kW16BlockSliceKT)) return;
  const int M = live_rows(counts, X::kRows);
  if (M == 0) return;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int out_tile = cg * WAVES + wave;
  const bool active = out_tile < tiles;  // a partial last group has idle waves
  int t = active ? out_tile : 0;
  const uint8_t *region[NW];
  region[0] = w0;
  if (MODE == 1) {
    if (t >= tq + tk) {
      region[0] = w2;
      t -= tq + tk;
    } else if (t >= tq) {
      region[0] = w1;
      t -= tq;
    }
  }
  if (NW == 2) region[NW - 1] = w1;
  const uint8_t *strip[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    strip[i] = expert_tiles(region[i], 0) + static_cast<uint64_t>(t) * KT * kTileBytes;
  }

  // 0. Channel scales of this lane's column (first: waits for the activation
  //    loads below never wait for them). Block scales: the epilogue's
  //    multiplier is 1 and the slice's k-tile scales of this wave's block
  //    (t / 8) go to LDS.
  float sc[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if constexpr (BLOCK) {
      sc[i] = 1.0f;
      const float *bs = expert_scales(region[i], 0) + static_cast<uint64_t>(t >> 3) * KT + kt0;
      for (int kl = lane; kl < nkt; kl += 64) bscale[(wave * NW + i) * kW16BlockSliceKT + kl] = bs[kl];
    } else {
      sc[i] = expert_scales(region[i], 0)[t * 16 + r];
    }
  }

  // Activation chunk c (k-tiles c XC .. c XC + XC - 1 of the slice) goes straight
  // into ring buffer c & 1 with global_load_lds: 1 KiB = 4 rows of one k-tile
  // per instruction, only the ceil(M / 4) row groups that hold live rows
  // (rows past M re-read row M - 1; their outputs are never stored).
  const uint32_t ring_base = __builtin_amdgcn_readfirstlane(w8a8v3::lds_offset_of(ring));
  const int xins = (M + 3) >> 2;
  const int chunks = (nkt + XC - 1) / XC;
  auto load_chunk = [&](int c) {
    const int n = (nkt - c * XC < XC ? nkt - c * XC : XC) * xins;
    for (int id = wave; id < n; id += WAVES) {
      const int kl = id / xins, q = id - kl * xins;
      const int row = 4 * q + (lane >> 4);
      const int chunk = (lane & 15) ^ chunk_swizzle(row);
      const int src = row < M ? row : M - 1;
      w8a8v3::dma16(reinterpret_cast<const uint8_t *>(x + static_cast<uint64_t>(src) * K +
                                                      (kt0 + c * XC + kl) * 128 + chunk * 8),
                    ring_base + (c & 1) * X::kBufferBytes + kl * X::kKTileBytes + q * 1024);
    }
  };
  // Weight loads issued after chunk c's activation loads and before the wait
  // for them: the refills of chunk c - 1 (one k-tile each while k-tiles
  // remain), i.e. 2 NW per refilled k-tile.
  auto refills = [&](int c) {
    const int n = nkt - D - c * XC;
    return n < 0 ? 0 : n > XC ? XC : n;
  };

  load_chunk(0);
  // Weight ring, D k-tiles deep.
  uint4 b[D][NW][2];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (d < nkt) load_tiles<NW>(strip, kt0 + d, lane, b[d]);
  }
  wait_vm_multiple<2 * NW, D>(nkt < D ? nkt : D);

  f32x4 acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Rows >= M of the ring hold stale LDS contents; they only feed output
  // rows >= M, which are never stored (MFMA rows are independent).
  for (int base = 0; base < nkt; base += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int kl = base + d;
      if (kl >= nkt) break;
      if (d % XC == 0) {
        const int c = kl / XC;
        if (c > 0) {
          // This wave's share of chunk c landed: only the refills of chunk
          // c - 1 were issued after it.
          if (refills(c - 1) == XC) {
            w8a8v3::wait_vmcnt<2 * NW * XC>();
          } else {
            w8a8v3::wait_vmcnt<0>();
          }
        }
        // Every wave's share of chunk c is in LDS, and every wave is done
        // with chunk c - 1, whose buffer chunk c + 1 now refills.
        __syncthreads();
        if (c + 1 < chunks) load_chunk(c + 1);
      }
      const uint8_t *buf = ring + ((kl / XC) & 1) * X::kBufferBytes + (d % XC) * X::kKTileBytes;
      // BLOCK: this k-tile's products, scaled into acc after its 4 MFMAs
      f32x4 part[BLOCK ? MT : 1][NW];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Frag16 a[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = mt * 16 + r;
          a[mt].u = *reinterpret_cast<const uint4 *>(
              buf + row * 256 + ((((g << 2) | j) ^ chunk_swizzle(row)) << 4));
        }
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          const bf16x8 bf = weight_fragment(b[d][i], j);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if constexpr (BLOCK) {
              part[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  a[mt].v, bf, j == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : part[mt][i], 0, 0, 0);
            } else {
              acc[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt].v, bf, acc[mt][i], 0, 0, 0);
            }
          }
        }
      }
      if constexpr (BLOCK) {
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          const float sb = bscale[(wave * NW + i) * kW16BlockSliceKT + kl];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[mt][i] += part[mt][i] * sb;
            // Keeps these reads of the MFMA results in the MFMAs' basic
            // block: sunk past the conditional refill below (as the compiler
            // otherwise does), the first read at the join was issued one
            // instruction after the last MFMA on the path that skips the
            // refill, with none of the wait states an MFMA result needs
            // before a VALU reads it (measured: element 3 of each fragment
            // varied from launch to launch at 16 rows).
            asm volatile("" : "+v"(acc[mt][i]));
          }
        }
      }
      if (kl + D < nkt) load_tiles<NW>(strip, kt0 + kl + D, lane, b[d]);
    }
  }

  group_epilogue<MT, NW, MODE>(acc, sc, M, S, s, cg, tiles, out_tile, active, ld, y, ws, last_block);
}

// ---------------------------------------------------------------------------
// One-tile form: a block owns one 16-column tile (NW weights) and its KS waves
// split K into contiguous ranges; no workspace, no cross-block reduction.
// A fragments are read straight from global memory (x is small and stays in
// L2), DA k-tiles ahead of use; weight k-tiles D ahead. The KS partial tiles
// are summed in LDS in wave order (deterministic).
// ---------------------------------------------------------------------------
template <int KS, int MT, int MODE, int D, int DA>
__device__ __forceinline__ void w8a16_tile_kernel(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                                  const uint8_t *w1, const uint8_t *w2, uint16_t *y) {
  constexpr int NW = MODE == 2 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) f32x4 red[KS][MT * NW][64];
  const WeightHeader &h0 = header_of(w0);
  if (!dense_regions_ok<MODE>(w0, w1, w2)) return;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = MODE == 1 ? static_cast<int>(h0.rows + header_of(w1).rows + header_of(w2).rows)
                           : static_cast<int>(h0.rows);
  const int out_tile = blockIdx.x;
  if (out_tile >= (ld >> 4)) return;
  const int M = live_rows(counts, 16 * MT);
  if (M == 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  int t = out_tile;
  const uint8_t *region[NW];
  region[0] = w0;
  if (MODE == 1) {
    if (t >= tq + tk) {
      region[0] = w2;
      t -= tq + tk;
    } else if (t >= tq) {
      region[0] = w1;
      t -= tq;
    }
  }
  if (NW == 2) region[NW - 1] = w1;
  const uint8_t *strip[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    strip[i] = expert_tiles(region[i], 0) + static_cast<uint64_t>(t) * KT * kTileBytes;
  }
  // Channel scales of the column this thread finishes in the epilogue
  // ((e >> 2) & 15 for its elements e = threadIdx.x + 64 KS i).
  const int ec = (threadIdx.x >> 2) & 15;
  float sc[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) sc[i] = expert_scales(region[i], 0)[t * 16 + ec];

  const int kt0 = (KT * wave) / KS, kt1 = (KT * (wave + 1)) / KS;
  const int nkt = kt1 - kt0;
  // This lane's A rows (rows past M re-read row M - 1; their outputs are
  // never stored).
  const uint16_t *xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = mt * 16 + r;
    xrow[mt] = x + static_cast<uint64_t>(row < M ? row : M - 1) * K + g * 32;
  }
  auto load_a = [&](int kt, uint4 (&dst)[MT][4]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint4 *p = reinterpret_cast<const uint4 *>(xrow[mt] + kt * 128);
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[mt][j] = p[j];
    }
  };
  uint4 b[D][NW][2];
  uint4 a[DA][MT][4];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (d < nkt) load_tiles<NW>(strip, kt0 + d, lane, b[d]);
    if (d < DA && d < nkt) load_a(kt0 + d, a[d]);
  }
  f32x4 acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  static_assert(D % DA == 0, "the A ring divides the weight ring");
  for (int base = 0; base < nkt; base += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int kl = base + d;
      if (kl < nkt) {
        uint4(&ad)[MT][4] = a[d % DA];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int i = 0; i < NW; ++i) {
            const bf16x8 bf = weight_fragment(b[d][i], j);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              Frag16 af;
              af.u = ad[mt][j];
              acc[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af.v, bf, acc[mt][i], 0, 0, 0);
            }
          }
        }
        if (kl + D < nkt) load_tiles<NW>(strip, kt0 + kl + D, lane, b[d]);
        if (kl + DA < nkt) load_a(kt0 + kl + DA, ad);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) red[wave][mt * NW + i][lane] = acc[mt][i];
  __syncthreads();
  // Element e of the tile: row tile mt, lane l, register rr (16x16 MFMA
  // accumulator layout: row 4 (l / 16) + rr, column l % 16).
  for (int e = threadIdx.x; e < MT * 256; e += KS * 64) {
    const int mt = e >> 8, l = (e >> 2) & 63, rr = e & 3;
    const int m = mt * 16 + 4 * (l >> 4) + rr;
    if (m >= M) continue;
    float v[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      float sum = 0.0f;
#pragma unroll
      for (int wv = 0; wv < KS; ++wv) sum += red[wv][mt * NW + i][l][rr];
      v[i] = sum;
    }
    const float out = MODE == 2 ? silu_mul(v[0] * sc[0], v[NW - 1] * sc[NW - 1]) : v[0] * sc[0];
    y[static_cast<uint64_t>(m) * ld + out_tile * 16 + ec] = static_cast<uint16_t>(f32_to_bf16(out));
  }
}

// The compiled shape of a specialized entry against a weight region's
// header. Read together with the live row count, right after the weight
// prologue is issued, so the scalar loads overlap the weight stream; read
// after the main loop (where it is used) it put a cold header fetch of
// about 1 us between the last MFMA and the stores.
// The first 32 header bytes are read in one go and compared without
// short-circuits, so the scalar loads issue together (a chain of && made the
// compiler fetch field by field, each after the previous comparison).
template <int NW, int K, uint32_t SCALE = kScalePerChannel>
LF_DEVICE bool fixed_shape_ok(const uint8_t *const (&region)[NW], int region_rows) {
  uint32_t bad = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const u32x4 *h = reinterpret_cast<const u32x4 *>(region[i]);
    const u32x4 a = h[0], b = h[1];  // magic, version, layout, scale_mode | rows, columns, experts
    bad |= (a.x ^ kWeightMagic) | (a.w ^ SCALE) |
           (b.x ^ static_cast<uint32_t>(region_rows)) | (b.y ^ static_cast<uint32_t>(K)) | (b.z ^ 1u);
  }
  return bad == 0;
}

// Block scales of the specialized forms (BLOCK): the scales of a region
// follow its tiles (the offset the header gives, computed from the compiled
// shape so no header read sits before the loads), [rows / 128][K / 128]. A
// wave's 16-column tile t lies in 128-row block t / 8; lane l of the
// returned value holds the scale of k-tile kt0 + l for l < n (n <= 64), so
// k-step k takes it with one readlane.
template <int K>
LF_DEVICE float block_scale_lanes(const uint8_t *region, int region_rows, int t, int kt0, int n) {
  constexpr int KT = K / 128;
  const float *s = reinterpret_cast<const float *>(region + kWeightHeaderBytes +
                                                   static_cast<uint64_t>(region_rows) * K) +
                   static_cast<uint64_t>(t >> 3) * KT + kt0;
  const int lane = threadIdx.x & 63;
  return lane < n ? s[lane] : 0.0f;
}
LF_DEVICE float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// ---------------------------------------------------------------------------
// Shape-specialized one-tile form. The input width K (and, for QKV, the Q and
// K/V widths) is a compile-time constant, as in an AOT entry point built for
// one model shape; the output width comes from the grid (one block per
// 16-column tile). Nothing on the load path waits for the weight header: the
// block issues its weight k-tiles the moment it starts, and checks the header
// against the compiled shape only before it stores.
//
// A block of KS waves owns one output tile (NW weights: gate and up for
// gate/up); wave w owns k-tiles [w KTW, (w + 1) KTW). Each wave keeps DW
// weight k-tiles and DX activation k-tiles in flight in registers. The loop
// over its KTW k-tiles is fully unrolled and branch-free, and the loads of
// step k + DX (activation) and k + DW (weights) are issued right after step
// k's MFMAs, activations first, so each step waits only for loads issued DX
// steps earlier: the compiler's s_waitcnt counts are exact and the weight
// stream never drains between k-tiles. (A rolled loop with conditional
// refills makes the compiler fall back to vmcnt(0) at every step, which
// serializes the ring.) The KS partial tiles are summed in LDS in wave order.
// ---------------------------------------------------------------------------
// BLOCK: weights with 128 x 128 block scales; each k-tile's MFMAs run into
// fresh fragments that are multiplied by the k-tile's block scale and added
// to the sums (the fold of w8a16_kernel's BLOCK form), no channel scale.
template <int K, int KS, int MT, int MODE, int DW, int DX, int NQ = 0, int NKV = 0, int SLOTS = 2,
          bool BLOCK = false>
__device__ __forceinline__ void w8a16_fixed_kernel(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                                   const uint8_t *w1, const uint8_t *w2, uint16_t *y) {
  constexpr int NW = MODE == 2 ? 2 : 1;
  constexpr int KT = K / 128;
  static_assert(K % 128 == 0 && KT % KS == 0, "K splits evenly over the waves");
  constexpr int KTW = KT / KS;
  constexpr int EW = DW < KTW ? DW : KTW;
  constexpr int EX = DX < EW ? DX : EW;
  constexpr int XI = 4 * MT;  // 1 KiB activation loads per k-tile (4 rows each)
  static_assert(MODE != 1 || (NQ % 16 == 0 && NKV % 16 == 0 && NQ > 0 && NKV > 0), "qkv widths");
  // Per wave: SLOTS k-tile slots of 16 MT activation rows (256 bytes each;
  // row r keeps 16-byte chunk c at position c ^ chunk_swizzle(r), so both the
  // row-wise writes and the 16-row fragment reads hit distinct banks). With
  // one slot, step k + 1's writes queue behind step k's fragment reads (a
  // wave's LDS instructions execute in order). The partial tiles of the K
  // reduction reuse the same memory after the main loop.
  static_assert(SLOTS == 1 || SLOTS == 2, "activation slots");
  constexpr int kSlot = 16 * MT * 16;  // 16-byte chunks per slot
  constexpr int kXsBytes = KS * SLOTS * kSlot * 16;
  constexpr int kRedBytes = KS * MT * NW * 64 * 16;
  __shared__ __attribute__((aligned(16))) u32x4 smem[(kXsBytes > kRedBytes ? kXsBytes : kRedBytes) / 16];
  u32x4 *xs = smem + wave_index() * SLOTS * kSlot;
  f32x4 *red = reinterpret_cast<f32x4 *>(smem);

  const int tiles = static_cast<int>(gridDim.x);
  const int out_tile = static_cast<int>(blockIdx.x);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int ld = MODE == 1 ? NQ + 2 * NKV : 16 * tiles;

  int t = out_tile;
  const uint8_t *region[NW];
  int region_rows = 16 * tiles;
  region[0] = w0;
  if constexpr (MODE == 1) {
    constexpr int tq = NQ / 16, tk = NKV / 16;
    region_rows = NQ;
    if (t >= tq + tk) {
      region[0] = w2;
      t -= tq + tk;
      region_rows = NKV;
    } else if (t >= tq) {
      region[0] = w1;
      t -= tq;
      region_rows = NKV;
    }
  }
  if constexpr (NW == 2) region[NW - 1] = w1;
  const uint64_t tile_base = kWeightHeaderBytes + static_cast<uint64_t>(t) * KT * kTileBytes;
  const uint8_t *strip[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) strip[i] = region[i] + tile_base;

  // Channel scales of the column this thread finishes in the epilogue:
  // per-channel scales follow the N x K tile block. BLOCK: the multiplier is
  // 1, and bsv[i] holds this wave's KTW k-tile scales, one per lane.
  const int ec = (threadIdx.x >> 2) & 15;
  const int kt0 = wave * KTW;
  float sc[NW], bsv[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if constexpr (BLOCK) {
      sc[i] = 1.0f;
      bsv[i] = block_scale_lanes<K>(region[i], region_rows, t, kt0, KTW);
    } else {
      sc[i] = reinterpret_cast<const float *>(
          region[i] + kWeightHeaderBytes + static_cast<uint64_t>(region_rows) * K)[t * 16 + ec];
    }
  }

  uint4 b[EW][NW][2];
#pragma unroll
  for (int d = 0; d < EW; ++d) load_tiles<NW>(strip, kt0 + d, lane, b[d]);
  // sched_barrier pins the issue order written here: the scheduler would
  // otherwise sink each load to just before its use to save registers,
  // which leaves only a k-tile or two in flight.
  __builtin_amdgcn_sched_barrier(0);

  // A region whose header disagrees with the compiled shape (a wrong weight
  // bound to this entry) counts as no live rows: nothing is stored.
  const int M = live_rows(counts, 16 * MT) &
                -static_cast<int>(fixed_shape_ok<NW, K, BLOCK ? kScaleBlock128 : kScalePerChannel>(
                    region, region_rows));
  // Activation loads are row-coalesced: instruction q gives lane l row
  // 4 q + l / 16, 16-byte chunk l % 16 of the k-tile (rows past M re-read row
  // M - 1; their outputs are never stored. M == 0 stores nothing).
  const uint16_t *xsrc[XI];
  int xdst[XI];
#pragma unroll
  for (int q = 0; q < XI; ++q) {
    const int row = 4 * q + (lane >> 4);
    const int src = row < M ? row : (M > 0 ? M - 1 : 0);
    xsrc[q] = x + static_cast<uint64_t>(src) * K + kt0 * 128 + (lane & 15) * 8;
    xdst[q] = row * 16 + ((lane & 15) ^ chunk_swizzle(row));
  }
  auto load_a = [&](int k, u32x4 (&dst)[XI]) {
#pragma unroll
    for (int q = 0; q < XI; ++q) dst[q] = *reinterpret_cast<const u32x4 *>(xsrc[q] + k * 128);
  };
  u32x4 a[EX][XI];
#pragma unroll
  for (int d = 0; d < EX; ++d) load_a(d, a[d]);
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  static_for<KTW>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    u32x4 *slot = xs + (k % SLOTS) * kSlot;
#pragma unroll
    for (int q = 0; q < XI; ++q) slot[xdst[q]] = a[k % EX][q];
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (k + EX < KTW) load_a(k + EX, a[k % EX]);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 part[BLOCK ? MT : 1][NW];  // BLOCK: this k-tile's products
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8 af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        af[mt] = __builtin_bit_cast(bf16x8, slot[(16 * mt + r) * 16 + (((g << 2) | j) ^ chunk_swizzle(r))]);
      }
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const bf16x8 bf = weight_fragment(b[k % EW][i], j);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (BLOCK) {
            part[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                af[mt], bf, j == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : part[mt][i], 0, 0, 0);
          } else {
            acc[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bf, acc[mt][i], 0, 0, 0);
          }
        }
      }
    }
    if constexpr (BLOCK) {
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const float sb = lane_value(bsv[i], k);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt][i] += part[mt][i] * sb;
          asm volatile("" : "+v"(acc[mt][i]));  // (in the MFMAs' block: w8a16_kernel)
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (k + EW < KTW) load_tiles<NW>(strip, kt0 + k + EW, lane, b[k % EW]);
    __builtin_amdgcn_sched_barrier(0);
  });

  __syncthreads();  // every wave is done with its activation slots
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) red[(wave * MT * NW + mt * NW + i) * 64 + lane] = acc[mt][i];
  __syncthreads();

  // Element e of the tile: row tile mt, lane l, register rr (16x16 MFMA
  // accumulator layout: row 4 (l / 16) + rr, column l % 16).
  for (int e = threadIdx.x; e < MT * 256; e += KS * 64) {
    const int mt = e >> 8, l = (e >> 2) & 63, rr = e & 3;
    const int m = mt * 16 + 4 * (l >> 4) + rr;
    if (m >= M) continue;
    float v[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      float sum = 0.0f;
#pragma unroll
      for (int wv = 0; wv < KS; ++wv) sum += red[(wv * MT * NW + mt * NW + i) * 64 + l][rr];
      v[i] = sum;
    }
    const float out = MODE == 2 ? silu_mul(v[0] * sc[0], v[NW - 1] * sc[NW - 1]) : v[0] * sc[0];
    y[static_cast<uint64_t>(m) * ld + out_tile * 16 + ec] = static_cast<uint16_t>(f32_to_bf16(out));
  }
}

// ---------------------------------------------------------------------------
// Shape-specialized column-group form: the split-K structure of
// w8a16_kernel (a block = WAVES adjacent 16-column tiles, one per wave, over
// one of S K-slices; partials reduced by group_epilogue) with the input
// width K and S compile-time, so each wave's loop over its K / (128 S)
// k-tiles is fully unrolled and branch-free and the compiler's s_waitcnt
// counts are exact (see w8a16_fixed_kernel). The activation k-tile (16 MT
// rows) is loaded cooperatively with row-coalesced 1 KiB loads into
// registers (ceil(XI / WAVES) loads per wave, DX k-tiles ahead), written to one of
// two LDS slots (chunk c of row r at c ^ chunk_swizzle(r)), and shared by the block's
// waves after one barrier per k-tile. The barrier waits only for LDS
// writes (no memory fence), so the weight ring stays in flight across it.
// ---------------------------------------------------------------------------
// No wait before the activation loads (see the one-launch GatedMlp below).
// A wait returns false when the block must not go on (it then loads no
// activation and stores nothing).
struct NoWait {
  LF_DEVICE bool operator()(int) const { return true; }
};

// bid / nblocks: the block's index and the block count of this kernel's
// part of the grid (default: blockIdx.x, gridDim.x). wait(s) runs after the
// weight prologue is in flight and before the first activation load of
// K-slice s; if it returns false the block returns there (no activation
// load, no store, no split-K arrival).
// KROT: each block walks its k-tiles starting at ((block / 8) mod NKT) and
// wrapping around, instead of at 0. Blocks are dispatched to the 8 XCDs in
// turn, so the blocks sharing one L2 start at different k-tiles. Unsplit
// forms (every block reads all of x) otherwise all read the same k-tile of
// x at the same moment from the same few L2 channels: gate/up at 32 rows
// 21.6 -> 20.5 us. The split-K forms read disjoint slices and were slower
// with it (down 17.8 -> 18.4 us), so they keep the plain order. The sums
// run in a different k order, so results differ from the plain order by
// fp32 rounding.
// BLOCK: 128 x 128 block scales, folded per k-tile as in w8a16_fixed_kernel.
template <int K, int S, int WAVES, int MT, int MODE, int DW, int DX, int NQ = 0, int NKV = 0,
          class Wait = NoWait, bool COHERENT_OUT = false, bool KROT = false, bool BLOCK = false>
__device__ __forceinline__ void w8a16_fixed_group_kernel(const int32_t *counts, const uint16_t *x,
                                         const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                         uint16_t *y, uint8_t *ws, int bid = -1, int nblocks = -1,
                                         const Wait &wait = Wait{}) {
  constexpr int NW = MODE == 2 ? 2 : 1;
  constexpr int KT = K / 128;
  static_assert(K % 128 == 0 && KT % S == 0, "K splits evenly into the slices");
  constexpr int NKT = KT / S;
  constexpr int EW = DW < NKT ? DW : NKT;
  constexpr int EX = DX < EW ? DX : EW;
  constexpr int XI = 4 * MT;
  // XPW = ceil(XI / WAVES) loads per wave, wave w taking loads w XPW .. + XPW
  // - 1 modulo XI. Where the waves' loads overrun XI (more waves than loads,
  // or XI not a multiple of WAVES) the later waves repeat the first rows:
  // identical values, so the duplicate LDS writes are benign.
  constexpr int XPW = (XI + WAVES - 1) / WAVES;
  static_assert(MODE != 1 || (NQ % 16 == 0 && NKV % 16 == 0 && NQ > 0 && NKV > 0), "qkv widths");
  constexpr int kSlot = 16 * MT * 16;  // 16-byte chunks per slot
  __shared__ __attribute__((aligned(16))) u32x4 xs[2 * kSlot];
  __shared__ int last_block;

  const int nb = nblocks < 0 ? static_cast<int>(gridDim.x) : nblocks;
  const int block = bid < 0 ? static_cast<int>(blockIdx.x) : bid;
  const int groups = nb / S;
  const int cg = block / S;
  const int s = block - cg * S;
  const int tiles = groups * WAVES;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int ld = MODE == 1 ? NQ + 2 * NKV : 16 * tiles;
  const int out_tile = cg * WAVES + wave;

  int t = out_tile;
  const uint8_t *region[NW];
  int region_rows = 16 * tiles;
  region[0] = w0;
  if constexpr (MODE == 1) {
    constexpr int tq = NQ / 16, tk = NKV / 16;
    region_rows = NQ;
    if (t >= tq + tk) {
      region[0] = w2;
      t -= tq + tk;
      region_rows = NKV;
    } else if (t >= tq) {
      region[0] = w1;
      t -= tq;
      region_rows = NKV;
    }
  }
  if constexpr (NW == 2) region[NW - 1] = w1;
  const int kt0 = s * NKT;
  // k-tile index of step k (KROT: rotated by the block's position on its XCD)
  const int rot = KROT ? __builtin_amdgcn_readfirstlane((block >> 3) % NKT) : 0;
  auto kr = [&](int k) {
    const int kk = k + rot;
    return kk < NKT ? kk : kk - NKT;
  };
  const uint64_t tile_base = kWeightHeaderBytes + static_cast<uint64_t>(t) * KT * kTileBytes;
  const uint8_t *strip[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) strip[i] = region[i] + tile_base;
  // BLOCK: the multiplier is 1, and bsv[i] holds this slice's NKT k-tile
  // scales, one per lane (NKT <= 64).
  static_assert(!BLOCK || NKT <= 64, "a slice's block scales fit one register");
  float sc[NW], bsv[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if constexpr (BLOCK) {
      sc[i] = 1.0f;
      bsv[i] = block_scale_lanes<K>(region[i], region_rows, t, kt0, NKT);
    } else {
      sc[i] = reinterpret_cast<const float *>(
          region[i] + kWeightHeaderBytes + static_cast<uint64_t>(region_rows) * K)[t * 16 + r];
    }
  }

  uint4 b[EW][NW][2];
#pragma unroll
  for (int d = 0; d < EW; ++d) load_tiles<NW>(strip, kt0 + kr(d), lane, b[d]);
  __builtin_amdgcn_sched_barrier(0);

  // A region whose header disagrees with the compiled shape counts as no
  // live rows: nothing is stored, and the block still takes part in the
  // split-K arrival count, so the counters stay consistent.
  const int M = live_rows(counts, 16 * MT) &
                -static_cast<int>(fixed_shape_ok<NW, K, BLOCK ? kScaleBlock128 : kScalePerChannel>(
                    region, region_rows));
  const uint16_t *xsrc[XPW];
  int xdst[XPW];
#pragma unroll
  for (int j = 0; j < XPW; ++j) {
    const int q = (wave * XPW + j) % XI;
    const int row = 4 * q + (lane >> 4);
    const int src = row < M ? row : (M > 0 ? M - 1 : 0);
    xsrc[j] = x + static_cast<uint64_t>(src) * K + kt0 * 128 + (lane & 15) * 8;
    xdst[j] = row * 16 + ((lane & 15) ^ chunk_swizzle(row));
  }
  auto load_a = [&](int k, u32x4 (&dst)[XPW]) {
#pragma unroll
    for (int j = 0; j < XPW; ++j) dst[j] = *reinterpret_cast<const u32x4 *>(xsrc[j] + kr(k) * 128);
  };
  if (!wait(s)) return;
  u32x4 a[EX][XPW];
#pragma unroll
  for (int d = 0; d < EX; ++d) load_a(d, a[d]);
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < NW; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  static_for<NKT>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    u32x4 *slot = xs + (k & 1) * kSlot;
#pragma unroll
    for (int j = 0; j < XPW; ++j) slot[xdst[j]] = a[k % EX][j];
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (k + EX < NKT) load_a(k + EX, a[k % EX]);
    // This wave's rows of k-tile k are in LDS; once every wave's are, the
    // slot is complete. (The other slot was last read at step k - 1, whose
    // fragment reads every wave consumed before this barrier.)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    f32x4 part[BLOCK ? MT : 1][NW];  // BLOCK: this k-tile's products
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8 af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        af[mt] = __builtin_bit_cast(bf16x8, slot[(16 * mt + r) * 16 + (((g << 2) | j) ^ chunk_swizzle(r))]);
      }
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const bf16x8 bf = weight_fragment(b[k % EW][i], j);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (BLOCK) {
            part[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                af[mt], bf, j == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : part[mt][i], 0, 0, 0);
          } else {
            acc[mt][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bf, acc[mt][i], 0, 0, 0);
          }
        }
      }
    }
    if constexpr (BLOCK) {
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const float sb = lane_value(bsv[i], kr(k));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt][i] += part[mt][i] * sb;
          asm volatile("" : "+v"(acc[mt][i]));  // (in the MFMAs' block: w8a16_kernel)
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (k + EW < NKT) load_tiles<NW>(strip, kt0 + kr(k + EW), lane, b[k % EW]);
    __builtin_amdgcn_sched_barrier(0);
  });

  group_epilogue<MT, NW, MODE, COHERENT_OUT>(acc, sc, M, S, s, cg, tiles, out_tile, true, ld, y, ws,
                               last_block);
}

// ---------------------------------------------------------------------------
// GatedMlp in one launch (x -> SiLU(x Wg^T) * (x Wu^T) -> h -> h Wd^T): the
// grid's first G1 blocks run the gate/up column-group kernel (K = H, split
// 1) into h in the workspace, the next G2 blocks the down column-group
// kernel (K = I, split DN_S) on h. Down K-slice s needs the h columns of
// G1 / DN_S gate/up blocks, which write h with agent-scope stores (through
// the XCD's L2; each 128-byte line of h has one writer) and count
// themselves into sync[s] once every wave's stores have completed - the
// pattern of the split-K exchange. A down block starts its weight ring,
// then one lane polls sync[s] before the block loads h: no block on the down
// block's XCD has read those lines of h in this launch (each is read only
// after its slice is complete), so the loads miss to memory and see the
// written values. (L2-wide write-back and invalidate fences in their place
// tripled the operation's time.)
//
// Measured on MI355X (Llama-3-8B widths, weights rotated past the MALL),
// this form runs as fast as the two launches it replaces at M = 32 (37.1
// vs 37.2 us) and 3 us behind them at M <= 16 (35.1 vs 32.0 us, where the
// two-launch path runs down on the faster one-tile form). Back-to-back
// launches on one queue cost almost nothing at the boundary, and the down
// part cannot start before the last gate/up block of its slice, so the one
// launch buys no overlap. It is the plan's entry for the operation (one
// launch per operation).
//
// Blocks are dispatched in index order on each XCD, so every gate/up block
// has a CU before any down block of its XCD takes one, and gate/up blocks
// wait for nothing: the polls end. They are bounded all the same
// (phases.h: about 2^20 polls, far beyond any real wait): one that runs out
// sets the error word, and its block returns without loading h or storing
// anything. The last down block to finish resets the slice counters and its
// own done counter for the next launch, unless the error word is set; every
// down block's wait reads the word with its first poll and fails while it
// is set, so a workspace whose counters are not at rest produces no output
// until the caller zero-fills it (the host binding does so when it reads
// the word after a synchronous launch).
//
// Workspace: h [16 MT rows][I] bf16 | the down kernel's split-K partials
// and arrival counters | sync (768 bytes): slice counter s at +128 s (a line
// each: phases.h), done (+512 B), error (+640 B, the last line but one; 0
// after every correct launch).
struct SliceWait {
  int *counters;
  int target;
  int *error;
  phase::Flag *flag;
  LF_DEVICE bool operator()(int s) const {
    return phase::wait_for(counters + phase::kLineInts * s, target, error, *flag);
  }
};

// BLOCK: all three weights carry 128 x 128 block scales.
template <int H, int I, int MT, int GU_W, int GU_DW, int GU_DX, int DN_S, int DN_W, int DN_DW,
          int DN_DX, bool BLOCK = false>
struct GatedMlpFixed {
  static constexpr int kG1 = I / 16 / GU_W;
  static constexpr int kG2 = H / 16 / DN_W * DN_S;
  static constexpr int kSliceCols = I / DN_S;
  static_assert(kSliceCols % (GU_W * 16) == 0 && kSliceCols % 128 == 0, "slices of whole blocks");
  static constexpr uint64_t kHBytes = (16ull * MT * I * 2 + 255) & ~255ull;
  static constexpr uint64_t kDownBytes =
      ((static_cast<uint64_t>(DN_S) * (H / 16) * MT * 1024 + 255) & ~255ull) +
      (((H / 16 / DN_W) * 4 + 255) & ~255ull);
  static constexpr uint64_t kSyncBytes = 768;
  static_assert(DN_S <= 4, "slice counters fit before the done word");

  LF_DEVICE static void run(const int32_t *counts, const uint16_t *x, const uint8_t *wg,
                            const uint8_t *wu, const uint8_t *wd, uint16_t *y, uint8_t *ws) {
    __shared__ phase::Flag flag;
    uint16_t *h = reinterpret_cast<uint16_t *>(ws);
    uint8_t *ws_down = ws + kHBytes;
    // The block ranges and tile indices below are compiled for a grid of
    // kG1 + kG2 blocks (the geometry's); any other grid stores and loads
    // nothing (a larger one would address tiles past the weight regions).
    if (static_cast<int>(gridDim.x) != kG1 + kG2) return;
    int *sync = reinterpret_cast<int *>(ws + kHBytes + kDownBytes);
    int *done = sync + 4 * phase::kLineInts;
    int *error = sync + 5 * phase::kLineInts;
    const int b = static_cast<int>(blockIdx.x);
    if (b < kG1) {
      w8a16_fixed_group_kernel<H, 1, GU_W, MT, 2, GU_DW, GU_DX, 0, 0, NoWait, true, true, BLOCK>(
          counts, x, wg, wu, wu, h, ws_down, b, kG1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(sync + phase::kLineInts * ((b * GU_W * 16) / kSliceCols), 1,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
    const SliceWait wait{sync, kSliceCols / (GU_W * 16), error, &flag};
    w8a16_fixed_group_kernel<I, DN_S, DN_W, MT, 0, DN_DW, DN_DX, 0, 0, SliceWait, false, false, BLOCK>(
        counts, h, wd, wd, wd, y, ws_down, b - kG1, kG2, wait);
    if (threadIdx.x == 0) {
      const int before = __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == kG2 - 1 && phase::load_agent(error) == 0) {
        for (int s = 0; s < DN_S; ++s) phase::store_agent(sync + phase::kLineInts * s, 0);
        phase::store_agent(done, 0);
      }
    }
  }
};

}  // namespace

#ifndef LF_W16_WAVES
#define LF_W16_WAVES 4
#endif

extern "C" {

#define LF_W8A16_ENTRIES(MT, M, D, XC)                                                              \
  __global__ __launch_bounds__(LF_W16_WAVES * 64) void lf_fp8_w8a16_dense_m##M(              \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) { \
    w8a16_kernel<LF_W16_WAVES, MT, 0, D, XC>(counts, x, w, w, w, y, ws);              \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16_WAVES * 64) void lf_fp8_w8a16_qkv_m##M(                \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,        \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                         \
    w8a16_kernel<LF_W16_WAVES, MT, 1, D, XC>(counts, x, wq, wk, wv, y, ws);           \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16_WAVES * 64) void lf_fp8_w8a16_gate_up_m##M(            \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,        \
      uint16_t *h, uint8_t *ws) {                                                            \
    w8a16_kernel<LF_W16_WAVES, MT, 2, D, XC>(counts, x, wg, wu, wu, h, ws);           \
  }

LF_W8A16_ENTRIES(1, 16, 4, 4)
LF_W8A16_ENTRIES(2, 32, 4, 4)
LF_W8A16_ENTRIES(4, 64, 4, 4)
LF_W8A16_ENTRIES(8, 128, 2, 2)

// The same column-group forms over weights with 128 x 128 block scales.
#define LF_W8A16_B128_ENTRIES(MT, M, D, XC)                                                     \
  __global__ __launch_bounds__(LF_W16_WAVES * 64) void lf_fp8_w8a16_dense_b128_m##M(         \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) { \
    w8a16_kernel<LF_W16_WAVES, MT, 0, D, XC, true>(counts, x, w, w, w, y, ws);               \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16_WAVES * 64) void lf_fp8_w8a16_qkv_b128_m##M(           \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,        \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                         \
    w8a16_kernel<LF_W16_WAVES, MT, 1, D, XC, true>(counts, x, wq, wk, wv, y, ws);            \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16_WAVES * 64) void lf_fp8_w8a16_gate_up_b128_m##M(       \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,        \
      uint16_t *h, uint8_t *ws) {                                                            \
    w8a16_kernel<LF_W16_WAVES, MT, 2, D, XC, true>(counts, x, wg, wu, wu, h, ws);            \
  }

LF_W8A16_B128_ENTRIES(1, 16, 4, 4)
LF_W8A16_B128_ENTRIES(2, 32, 4, 4)
LF_W8A16_B128_ENTRIES(4, 64, 4, 4)
LF_W8A16_B128_ENTRIES(8, 128, 2, 2)

#ifndef LF_W16T_WAVES
#define LF_W16T_WAVES 8
#endif
#define LF_W8A16_TILE_ENTRIES(MT, M, DA)                                                      \
  __global__ __launch_bounds__(LF_W16T_WAVES * 64) void lf_fp8_w8a16_dense_m##M##_t1(        \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *) {  \
    w8a16_tile_kernel<LF_W16T_WAVES, MT, 0, 4, DA>(counts, x, w, w, w, y);                    \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16T_WAVES * 64) void lf_fp8_w8a16_qkv_m##M##_t1(          \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,        \
      const uint8_t *wv, uint16_t *y, uint8_t *) {                                           \
    w8a16_tile_kernel<LF_W16T_WAVES, MT, 1, 4, DA>(counts, x, wq, wk, wv, y);                 \
  }                                                                                          \
  __global__ __launch_bounds__(LF_W16T_WAVES * 64) void lf_fp8_w8a16_gate_up_m##M##_t1(      \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,        \
      uint16_t *h, uint8_t *) {                                                              \
    w8a16_tile_kernel<LF_W16T_WAVES, MT, 2, 4, DA>(counts, x, wg, wu, wu, h);                 \
  }

LF_W8A16_TILE_ENTRIES(1, 16, 1)

// Shape-specialized entries for Llama-3-8B (hidden 4096, intermediate
// 14336, Q 4096, K/V 1024): one-tile (t1) or column-group (g) form, chosen
// per (shape, profile) by lunaflux_fp8_launch_geometry; the parameters are
// the measured best of a sweep on MI355X (waves, weight / activation ring
// depth, LDS slots, K-slices). Gate/up has enough tiles (896) to fill the
// chip with unsplit column groups (2 or 4 tiles per block, S = 1): no
// exchange, and the activations are read once per group.
#define LF_W16_FIXED_DENSE_T1(KK, M, MT, KS, DW, DX, SLOTS)                                     \
  __global__ __launch_bounds__(KS * 64) void lf_fp8_w8a16_dense_k##KK##_m##M(                \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *) {  \
    w8a16_fixed_kernel<KK, KS, MT, 0, DW, DX, 0, 0, SLOTS>(counts, x, w, w, w, y);            \
  }
#define LF_W16_FIXED_QKV_T1(KK, NQ, NKV, M, MT, KS, DW, DX, SLOTS)                              \
  __global__ __launch_bounds__(KS * 64) void lf_fp8_w8a16_qkv_k##KK##_q##NQ##_kv##NKV##_m##M( \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,        \
      const uint8_t *wv, uint16_t *y, uint8_t *) {                                           \
    w8a16_fixed_kernel<KK, KS, MT, 1, DW, DX, NQ, NKV, SLOTS>(counts, x, wq, wk, wv, y);      \
  }
#define LF_W16_FIXED_QKV_G(KK, NQ, NKV, M, MT, S, W, DW, DX)                                    \
  __global__ __launch_bounds__(W * 64) void lf_fp8_w8a16_qkv_k##KK##_q##NQ##_kv##NKV##_m##M(  \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,        \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                         \
    w8a16_fixed_group_kernel<KK, S, W, MT, 1, DW, DX, NQ, NKV>(counts, x, wq, wk, wv, y, ws);  \
  }
#define LF_W16_FIXED_DENSE_G(KK, M, MT, S, W, DW, DX)                                           \
  __global__ __launch_bounds__(W * 64) void lf_fp8_w8a16_dense_k##KK##_m##M(                 \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) { \
    w8a16_fixed_group_kernel<KK, S, W, MT, 0, DW, DX>(counts, x, w, w, w, y, ws);             \
  }
// Wide dense shapes (the vocabulary head): unsplit column groups.
#define LF_W16_FIXED_DENSE_WIDE_G(KK, M, MT, S, W, DW, DX)                                      \
  __global__ __launch_bounds__(W * 64) void lf_fp8_w8a16_dense_wide_k##KK##_m##M(            \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) { \
    w8a16_fixed_group_kernel<KK, S, W, MT, 0, DW, DX, 0, 0, NoWait, false, S == 1>(            \
        counts, x, w, w, w, y, ws);                                                          \
  }
#define LF_W16_FIXED_GATE_UP_G(KK, M, MT, S, W, DW, DX)                                         \
  __global__ __launch_bounds__(W * 64) void lf_fp8_w8a16_gate_up_k##KK##_m##M(               \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,        \
      uint16_t *h, uint8_t *ws) {                                                            \
    w8a16_fixed_group_kernel<KK, S, W, MT, 2, DW, DX, 0, 0, NoWait, false, S == 1>(            \
        counts, x, wg, wu, wu, h, ws);                                                       \
  }

LF_W16_FIXED_DENSE_T1(4096, 16, 1, 8, 4, 2, 2)
LF_W16_FIXED_DENSE_T1(4096, 32, 2, 8, 4, 1, 1)
LF_W16_FIXED_DENSE_T1(14336, 16, 1, 8, 6, 2, 2)
LF_W16_FIXED_DENSE_G(14336, 32, 2, 4, 4, 6, 2)
LF_W16_FIXED_QKV_T1(4096, 4096, 1024, 16, 1, 8, 4, 2, 2)
LF_W16_FIXED_QKV_G(4096, 4096, 1024, 32, 2, 4, 8, 4, 2)
LF_W16_FIXED_GATE_UP_G(4096, 16, 1, 1, 2, 4, 2)
LF_W16_FIXED_GATE_UP_G(4096, 32, 2, 1, 4, 3, 2)
// Profiles of 65..128 rows use the LDS-tiled GEMM (w8a16_gemm.hip), except
// for these wide shapes.
// N >= 16384 (e.g. the 128,256-wide vocabulary head): enough 16-column
// tiles to fill the chip without a K split, as gate/up.
LF_W16_FIXED_DENSE_WIDE_G(4096, 16, 1, 1, 2, 4, 2)
LF_W16_FIXED_DENSE_WIDE_G(4096, 32, 2, 1, 4, 3, 2)
LF_W16_FIXED_DENSE_WIDE_G(4096, 128, 8, 1, 8, 2, 1)

// One-launch GatedMlp, Llama-3-8B widths (H 4096, I 14336), operands
// (counts, x, wg, wu, wd, y, ws): the profile's gate/up and down column-group
// parameters (blocks of GU_W = DN_W waves).
#define LF_W16_GATED_MLP(M, MT, GU_W, GU_DW, GU_DX, DN_S, DN_W, DN_DW, DN_DX)                     \
  __global__ __launch_bounds__(64 * GU_W) void lf_fp8_w8a16_gated_mlp_h4096_i14336_m##M(        \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      const uint8_t *wd, uint16_t *y, uint8_t *ws) {                                             \
    static_assert(GU_W == DN_W, "one block size");                                              \
    GatedMlpFixed<4096, 14336, MT, GU_W, GU_DW, GU_DX, DN_S, DN_W, DN_DW, DN_DX>::run(           \
        counts, x, wg, wu, wd, y, ws);                                                           \
  }

LF_W16_GATED_MLP(16, 1, 4, 4, 2, 4, 4, 6, 2)
LF_W16_GATED_MLP(32, 2, 4, 3, 2, 4, 4, 6, 2)

// The specialized entries over weights with 128 x 128 block scales
// (lf_fp8_w8a16_{op}_b128_k..., lf_fp8_w8a16_gated_mlp_b128_h4096_i14336_mM):
// the same forms and parameters with the per-k-tile fold.
#define LF_W16_FIXED_B128_DENSE_T1(KK, M, MT, KS, DW, DX, SLOTS)                                \
  __global__ __launch_bounds__(KS * 64) void lf_fp8_w8a16_dense_b128_k##KK##_m##M(           \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *) {  \
    w8a16_fixed_kernel<KK, KS, MT, 0, DW, DX, 0, 0, SLOTS, true>(counts, x, w, w, w, y);      \
  }
#define LF_W16_FIXED_B128_QKV_T1(KK, NQ, NKV, M, MT, KS, DW, DX, SLOTS)                         \
  __global__ __launch_bounds__(KS * 64) void                                                 \
      lf_fp8_w8a16_qkv_b128_k##KK##_q##NQ##_kv##NKV##_m##M(                                  \
          const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,    \
          const uint8_t *wv, uint16_t *y, uint8_t *) {                                       \
    w8a16_fixed_kernel<KK, KS, MT, 1, DW, DX, NQ, NKV, SLOTS, true>(counts, x, wq, wk, wv, y); \
  }
#define LF_W16_FIXED_B128_QKV_G(KK, NQ, NKV, M, MT, S, W, DW, DX)                               \
  __global__ __launch_bounds__(W * 64) void                                                  \
      lf_fp8_w8a16_qkv_b128_k##KK##_q##NQ##_kv##NKV##_m##M(                                  \
          const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,    \
          const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                     \
    w8a16_fixed_group_kernel<KK, S, W, MT, 1, DW, DX, NQ, NKV, NoWait, false, false, true>(    \
        counts, x, wq, wk, wv, y, ws);                                                       \
  }
#define LF_W16_FIXED_B128_DENSE_G(KK, M, MT, S, W, DW, DX)                                      \
  __global__ __launch_bounds__(W * 64) void lf_fp8_w8a16_dense_b128_k##KK##_m##M(            \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) { \
    w8a16_fixed_group_kernel<KK, S, W, MT, 0, DW, DX, 0, 0, NoWait, false, false, true>(       \
        counts, x, w, w, w, y, ws);                                                          \
  }
#define LF_W16_FIXED_B128_GATE_UP_G(KK, M, MT, S, W, DW, DX)                                    \
  __global__ __launch_bounds__(W * 64) void lf_fp8_w8a16_gate_up_b128_k##KK##_m##M(          \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,        \
      uint16_t *h, uint8_t *ws) {                                                            \
    w8a16_fixed_group_kernel<KK, S, W, MT, 2, DW, DX, 0, 0, NoWait, false, S == 1, true>(      \
        counts, x, wg, wu, wu, h, ws);                                                       \
  }
#define LF_W16_GATED_MLP_B128(M, MT, GU_W, GU_DW, GU_DX, DN_S, DN_W, DN_DW, DN_DX)                \
  __global__ __launch_bounds__(64 * GU_W) void lf_fp8_w8a16_gated_mlp_b128_h4096_i14336_m##M(   \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,            \
      const uint8_t *wd, uint16_t *y, uint8_t *ws) {                                             \
    static_assert(GU_W == DN_W, "one block size");                                              \
    GatedMlpFixed<4096, 14336, MT, GU_W, GU_DW, GU_DX, DN_S, DN_W, DN_DW, DN_DX, true>::run(     \
        counts, x, wg, wu, wd, y, ws);                                                           \
  }

LF_W16_FIXED_B128_DENSE_T1(4096, 16, 1, 8, 4, 2, 2)
LF_W16_FIXED_B128_DENSE_T1(4096, 32, 2, 8, 4, 1, 1)
LF_W16_FIXED_B128_DENSE_T1(14336, 16, 1, 8, 6, 2, 2)
LF_W16_FIXED_B128_DENSE_G(14336, 32, 2, 4, 4, 6, 2)
LF_W16_FIXED_B128_QKV_T1(4096, 4096, 1024, 16, 1, 8, 4, 2, 2)
LF_W16_FIXED_B128_QKV_G(4096, 4096, 1024, 32, 2, 4, 8, 4, 2)
LF_W16_FIXED_B128_GATE_UP_G(4096, 16, 1, 1, 2, 4, 2)
LF_W16_FIXED_B128_GATE_UP_G(4096, 32, 2, 1, 4, 3, 2)
LF_W16_GATED_MLP_B128(16, 1, 4, 4, 2, 4, 4, 6, 2)
LF_W16_GATED_MLP_B128(32, 2, 4, 3, 2, 4, 4, 6, 2)

}  // extern "C"
