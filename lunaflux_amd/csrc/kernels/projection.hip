// projection.hip - gfx950 kernels of the prefill regime: the per-token
// activation quantizer and the W8A8 FP8 MFMA GEMM (QKV, output/down,
// gate/up + SwiGLU). Entry points and operand lists are documented in
// include/lunaflux_fp8.h; every parameter is a device region.
#include "w8a8_v3.h"
#include "w8a8_v4.h"
#include "w8a8_v5.h"

namespace {

// ---------------------------------------------------------------------------
// Activation quantizers. For each span of columns (the whole row, or one
// 128-column group): amax over the span, ratio = 448 / amax (correctly
// rounded division), codes = e4m3_rne_sat(x * ratio), scale = amax / 448.
// An all-zero span gets zero codes and scale 0.
// ---------------------------------------------------------------------------
LF_DEVICE float bf16x8_amax(const uint4 &v, float amax) {
  const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    amax = fmaxf(amax, fabsf(bf16_to_f32(w4[i] & 0xffffu)));
    amax = fmaxf(amax, fabsf(bf16_to_f32(w4[i] >> 16)));
  }
  return amax;
}

// Four bf16 values (two words, element 2i in the low half of word i) times
// ratio -> four e4m3 codes, element j in byte j. v_cvt_pk_fp8_f32 rounds to
// nearest even (OCP E4M3: bias 7, max 448) and agrees bit for bit with a
// software round-to-nearest-even encoder that saturates to +-448 on every
// |v| <= 449 (checked on MI355X over 55 M inputs: every 7th fp32 in
// [2^-14, 512), subnormal outputs, each tie between codes +-2 ulp, both
// signs, NaN); above 464 it gives NaN where that encoder saturates. A
// quantizer's inputs x * (448 / amax) stay below 448 (1 + 2^-24)^2, so that
// range is never reached. All-zero spans (amax 0) get zero codes from the
// caller's select.
LF_DEVICE uint32_t e4m3x4_from_bf16(uint32_t w0, uint32_t w1, float ratio) {
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_to_f32(w0 & 0xffffu) * ratio,
                                          bf16_to_f32(w0 >> 16) * ratio, 0, false);
  p = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_to_f32(w1 & 0xffffu) * ratio,
                                      bf16_to_f32(w1 >> 16) * ratio, p, true);
  return static_cast<uint32_t>(p);
}

LF_DEVICE uint2 bf16x8_encode(const uint4 &v, float ratio, bool zero) {
  const uint32_t lo = e4m3x4_from_bf16(v.x, v.y, ratio);
  const uint32_t hi = e4m3x4_from_bf16(v.z, v.w, ratio);
  return make_uint2(zero ? 0u : lo, zero ? 0u : hi);
}

// The value of x as far as the compiler knows is whatever an empty asm left.
LF_DEVICE void opaque(u32x4 &x) { asm volatile("" : "+v"(x)); }

// Per-token quantizer, register-resident: one wave per row, lane l holding
// 16-byte chunks l, l + 64, ..., l + 64 (C - 1) (rows of up to 512 C
// columns), so the row is read from memory once with all of its loads in
// flight; then the wave's amax and the encode from registers.
// THROUGH: codes and scale are stored through the XCD's L2 (agent-scope
// atomic stores, phases.h), for rows that blocks of the same launch read.
template <bool THROUGH>
LF_DEVICE void store_codes8(uint8_t *p, uint32_t lo, uint32_t hi) {
  if constexpr (THROUGH) {
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), (static_cast<uint64_t>(hi) << 32) | lo,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<uint2 *>(p) = make_uint2(lo, hi);
  }
}
template <bool THROUGH>
LF_DEVICE void store_scale(float *p, float v) {
  if constexpr (THROUGH) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *p = v;
  }
}

// RB consecutive rows at once (rows row0 .. row0 + live - 1 of x, live <=
// RB): every load of the batch is issued before the first row is reduced,
// so a wave keeps RB rows in flight (RB C 16 bytes per lane). Returns the
// scale of the batch's first row.
template <int C, int RB, bool THROUGH = false>
LF_DEVICE float quantize_rows_wave_regs(const uint16_t *x, int K, int row0, int live, uint8_t *xq,
                                        float *scales) {
  const int lane = threadIdx.x & 63;
  const int chunks = K >> 3;
  u32x4 v[RB][C];
  static_for<RB>([&](auto b) {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(x + static_cast<uint64_t>(row0 + b) * K);
    static_for<C>([&](auto c) {
      const int idx = lane + 64 * c;
      v[b][c] = (b < live && idx < chunks) ? src[idx] : u32x4{0u, 0u, 0u, 0u};
    });
  });
  float first = 0.0f;
  static_for<RB>([&](auto b) {
    float amax = 0.0f;
    static_for<C>([&](auto c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        amax = fmaxf(amax, fabsf(bf16_to_f32(v[b][c][i] & 0xffffu)));
        amax = fmaxf(amax, fabsf(bf16_to_f32(v[b][c][i] >> 16)));
      }
    });
    amax = wave_max(amax);
    const bool zero = amax == 0.0f;
    const float ratio = zero ? 0.0f : 448.0f / amax;
    // The encode converts the raw chunks again rather than keeping the 8 C
    // floats of the amax pass alive (an empty asm that "redefines" each
    // chunk keeps the compiler from reusing them; 8 C floats would not fit).
    static_for<C>([&](auto c) { opaque(v[b][c]); });
    uint8_t *dst = xq + static_cast<uint64_t>(row0 + b) * K;
    static_for<C>([&](auto c) {
      const int idx = lane + 64 * c;
      const uint32_t lo = e4m3x4_from_bf16(v[b][c][0], v[b][c][1], ratio);
      const uint32_t hi = e4m3x4_from_bf16(v[b][c][2], v[b][c][3], ratio);
      if (b < live && idx < chunks) store_codes8<THROUGH>(dst + 8 * idx, zero ? 0u : lo, zero ? 0u : hi);
    });
    const float sc = zero ? 0.0f : amax / 448.0f;
    if (b < live && lane == 0) store_scale<THROUGH>(scales + row0 + b, sc);
    if (b == 0) first = sc;
  });
  return first;
}

template <int C, bool THROUGH = false>
LF_DEVICE float quantize_row_wave_regs(const uint16_t *src_row, int K, uint8_t *dst_row,
                                       float *scale) {
  return quantize_rows_wave_regs<C, 1, THROUGH>(src_row, K, 0, 1, dst_row, scale);
}

// Per-token quantizer for rows longer than the register-resident forms: two
// passes over the row (amax, then encode); the second re-reads it from cache.
template <bool THROUGH = false>
LF_DEVICE float quantize_row_wave_2pass(const uint16_t *src_row, int K, uint8_t *dst_row,
                                        float *scale) {
  const int lane = threadIdx.x & 63;
  const int chunks = K >> 3;  // 8 bf16 per 16-byte chunk
  const uint4 *src = reinterpret_cast<const uint4 *>(src_row);
  float amax = 0.0f;
#pragma unroll 8
  for (int c = lane; c < chunks; c += 64) amax = bf16x8_amax(src[c], amax);
  amax = wave_max(amax);
  const bool zero = amax == 0.0f;
  const float ratio = zero ? 0.0f : 448.0f / amax;
#pragma unroll 8
  for (int c = lane; c < chunks; c += 64) {
    const uint2 e = bf16x8_encode(src[c], ratio, zero);
    store_codes8<THROUGH>(dst_row + 8 * c, e.x, e.y);
  }
  const float sc = zero ? 0.0f : amax / 448.0f;
  if (lane == 0) store_scale<THROUGH>(scale, sc);
  return sc;
}

// One wave per row, the register-resident form sized for the row (K is
// wave-uniform, so the branch is too). Returns the row's scale in every
// lane after lane 0 has stored it. Same arithmetic in every form.
// MAXC: the widest register-resident form (chunks per lane) the caller's
// register budget allows; wider rows take the two-pass form.
template <bool THROUGH = false, int MAXC = 32>
LF_DEVICE float quantize_row_wave(const uint16_t *src_row, int K, uint8_t *dst_row,
                                  float *scale) {
  if (K <= 4096) return quantize_row_wave_regs<8, THROUGH>(src_row, K, dst_row, scale);
  if (MAXC >= 16 && K <= 8192) return quantize_row_wave_regs<16, THROUGH>(src_row, K, dst_row, scale);
  if (MAXC >= 32 && K <= 16384) return quantize_row_wave_regs<32, THROUGH>(src_row, K, dst_row, scale);
  return quantize_row_wave_2pass<THROUGH>(src_row, K, dst_row, scale);
}

// v of the lane that DPP control CTRL selects within this lane's row of 16
// (every lane of the wave active).
template <int CTRL>
LF_DEVICE float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Per-128-column-group quantizer: the 16 lanes 16q..16q+15 of a wave hold
// one group's 16 chunks, so a wave quantizes a quad of four groups (of the
// rows x (K / 128) groups, row-major) at a time, amax reduced across its 16
// lanes. Wave gw of nw takes quads gw, gw + nw, ...; the loads of eight quads
// are issued before any of them is encoded.
LF_DEVICE void quantize_groups_wave(const uint16_t *src, int K, int rows, uint8_t *dst,
                                    float *scales, int gw, int nw) {
  const int lane = threadIdx.x & 63;
  const int per_row = K >> 7;
  const int groups = rows * per_row;
  const int quads = (groups + 3) >> 2;
  constexpr int kBatch = 8;
  for (int q0 = gw; q0 < quads; q0 += kBatch * nw) {
    uint4 v[kBatch];
    uint64_t base[kBatch];
    int gid[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      gid[b] = 4 * (q0 + b * nw) + (lane >> 4);
      const bool live = gid[b] < groups;
      const int row = live ? gid[b] / per_row : 0, kg = live ? gid[b] - row * per_row : 0;
      base[b] = static_cast<uint64_t>(row) * K + kg * 128 + (lane & 15) * 8;
      v[b] = live ? *reinterpret_cast<const uint4 *>(src + base[b]) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      float amax = bf16x8_amax(v[b], 0.0f);
      // maximum over the 16 lanes of the DPP row: swaps within quads, then
      // the other quad of the half-row (mirror), then the other half-row
      // (mirror); register-to-register, where a shuffle goes through LDS.
      // The maximum is the same in any order.
      amax = fmaxf(amax, dpp_f32<0xB1>(amax));   // quad_perm [1, 0, 3, 2]
      amax = fmaxf(amax, dpp_f32<0x4E>(amax));   // quad_perm [2, 3, 0, 1]
      amax = fmaxf(amax, dpp_f32<0x141>(amax));  // row_half_mirror
      amax = fmaxf(amax, dpp_f32<0x140>(amax));  // row_mirror
      const bool zero = amax == 0.0f;
      const float ratio = zero ? 0.0f : 448.0f / amax;
      if (gid[b] < groups) {
        *reinterpret_cast<uint2 *>(dst + base[b]) = bf16x8_encode(v[b], ratio, zero);
        if ((lane & 15) == 0) scales[gid[b]] = zero ? 0.0f : amax / 448.0f;
      }
    }
  }
}

// One wave per row, four rows per block.
LF_DEVICE void act_quant_rows(const int32_t *counts, const uint16_t *x, const uint8_t *w,
                               uint8_t *xq) {
  const WeightHeader &h = header_of(w);
  if (h.magic != kWeightMagic) return;
  const int K = static_cast<int>(h.columns);
  const int M = live_rows(counts, 1 << 30);
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  float *scales = reinterpret_cast<float *>(xq + align256(static_cast<uint64_t>(M) * K));
  quantize_row_wave(x + static_cast<uint64_t>(row) * K, K, xq + static_cast<uint64_t>(row) * K,
                    scales + row);
}

// ---------------------------------------------------------------------------
// RmsNorm fused with the per-token quantizer (kernels/reference/basic.mbt:
// 32-68, then the quantizer above on the fp32 result): for row r
//   ss  = sum_k x[r, k]^2    fp32: each lane sums its own values in column
//                            order, then a xor butterfly across the wave
//   inv = 1 / sqrt(ss / K + eps)      correctly rounded sqrt and division, as
//                                     the reference's fp32 operations
//   y_k = (x[r, k] * inv) * g[k]      the reference's left-to-right order
// and the codes and scale of y as the quantizer forms them (amax, ratio =
// 448 / amax, e4m3_rne_sat(y * ratio), scale = amax / 448). Only the order of
// the sum of squares differs from the reference's sequential loop. A row whose
// sum of squares overflows (the reference raises NonFinite) gets inv = 0,
// hence zero codes and scale 0. One wave per row, register-resident as the
// quantizer: the row and the norm weight stay in registers (rows of up to
// 8192 columns).
// ---------------------------------------------------------------------------
LF_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset);
  return v;
}

LF_DEVICE float rms_scaled(uint32_t xbits, uint32_t gbits, float inv) {
  return __fmul_rn(__fmul_rn(bf16_to_f32(xbits), inv), bf16_to_f32(gbits));
}

// Four normalized values (x words x0, x1 and norm-weight words g0, g1) times
// ratio -> four e4m3 codes, element j in byte j.
LF_DEVICE uint32_t e4m3x4_from_norm(uint32_t x0, uint32_t x1, uint32_t g0, uint32_t g1, float inv,
                                    float ratio) {
  int p = __builtin_amdgcn_cvt_pk_fp8_f32(rms_scaled(x0 & 0xffffu, g0 & 0xffffu, inv) * ratio,
                                          rms_scaled(x0 >> 16, g0 >> 16, inv) * ratio, 0, false);
  p = __builtin_amdgcn_cvt_pk_fp8_f32(rms_scaled(x1 & 0xffffu, g1 & 0xffffu, inv) * ratio,
                                      rms_scaled(x1 >> 16, g1 >> 16, inv) * ratio, p, true);
  return static_cast<uint32_t>(p);
}

template <int C>
LF_DEVICE void rms_norm_quant_row_wave(const uint16_t *x_row, const uint16_t *gamma, int K,
                                       float eps, uint8_t *dst_row, float *scale) {
  const int lane = threadIdx.x & 63;
  const int chunks = K >> 3;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(x_row);
  const u32x4 *gsrc = reinterpret_cast<const u32x4 *>(gamma);
  u32x4 v[C], g[C];
  static_for<C>([&](auto c) {
    const int idx = lane + 64 * c;
    v[c] = idx < chunks ? src[idx] : u32x4{0u, 0u, 0u, 0u};
    g[c] = idx < chunks ? gsrc[idx] : u32x4{0u, 0u, 0u, 0u};
  });
  float ss = 0.0f;
  static_for<C>([&](auto c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_to_f32(v[c][i] & 0xffffu), hi = bf16_to_f32(v[c][i] >> 16);
      ss = __fadd_rn(ss, __fmul_rn(lo, lo));
      ss = __fadd_rn(ss, __fmul_rn(hi, hi));
    }
  });
  static_for<C>([&](auto c) { opaque(v[c]); });  // no x floats kept across passes
  ss = wave_sum(ss);
  // __builtin_sqrtf and '/' are the correctly rounded IEEE operations (hipcc's
  // default fp32 division and sqrt lowering); HIP's __fsqrt_rn is the native
  // approximate v_sqrt_f32 unless OCML's rounded operations are enabled.
  const float root = __builtin_sqrtf(__fadd_rn(ss / static_cast<float>(K), eps));
  const float inv = isinf(ss) ? 0.0f : 1.0f / root;
  float amax = 0.0f;
  static_for<C>([&](auto c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      amax = fmaxf(amax, fabsf(rms_scaled(v[c][i] & 0xffffu, g[c][i] & 0xffffu, inv)));
      amax = fmaxf(amax, fabsf(rms_scaled(v[c][i] >> 16, g[c][i] >> 16, inv)));
    }
  });
  amax = wave_max(amax);
  const bool zero = amax == 0.0f;
  const float ratio = zero ? 0.0f : 448.0f / amax;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  u32x2 *dst = reinterpret_cast<u32x2 *>(dst_row);
  // As in the quantizer, the encode converts the raw words again (the empty
  // asms keep the compiler from holding the 8 C products).
  static_for<C>([&](auto c) { opaque(v[c]); });
  static_for<C>([&](auto c) { opaque(g[c]); });
  static_for<C>([&](auto c) {
    const int idx = lane + 64 * c;
    const uint32_t lo = e4m3x4_from_norm(v[c][0], v[c][1], g[c][0], g[c][1], inv, ratio);
    const uint32_t hi = e4m3x4_from_norm(v[c][2], v[c][3], g[c][2], g[c][3], inv, ratio);
    if (idx < chunks) dst[idx] = u32x2{zero ? 0u : lo, zero ? 0u : hi};
  });
  if (lane == 0) *scale = zero ? 0.0f : amax / 448.0f;
}

// One wave per row, four rows per block; K from the header of w (the first
// weight of the projection the quantized rows feed), at most 8192.
LF_DEVICE void rms_norm_quant_rows(const int32_t *counts, const uint16_t *x,
                                   const uint16_t *gamma, const uint8_t *w, uint8_t *xq,
                                   float eps) {
  const WeightHeader &h = header_of(w);
  if (h.magic != kWeightMagic) return;
  const int K = static_cast<int>(h.columns);
  if (K > 8192) return;
  const int M = live_rows(counts, 1 << 30);
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  float *scales = reinterpret_cast<float *>(xq + align256(static_cast<uint64_t>(M) * K));
  const uint16_t *src = x + static_cast<uint64_t>(row) * K;
  uint8_t *dst = xq + static_cast<uint64_t>(row) * K;
  if (K <= 4096) {
    rms_norm_quant_row_wave<8>(src, gamma, K, eps, dst, scales + row);
  } else {
    rms_norm_quant_row_wave<16>(src, gamma, K, eps, dst, scales + row);
  }
}

// ---------------------------------------------------------------------------
// Pieces shared by the W8A8 GEMM bodies below.
// ---------------------------------------------------------------------------
// Gate of a GEMM tile: called with the tile's first row before any of its
// activation rows or row scales is read; false means the tile is not
// computed and nothing is stored (Open: every tile runs).
struct Open {
  LF_DEVICE bool operator()(int) const { return true; }
};

// Output row width: N (dense, gate/up: I) or Nq + Nk + Nv (QKV).
template <int MODE>
LF_DEVICE int dense_ld(const uint8_t *w0, const uint8_t *w1, const uint8_t *w2) {
  return MODE == 1 ? static_cast<int>(header_of(w0).rows + header_of(w1).rows + header_of(w2).rows)
                   : static_cast<int>(header_of(w0).rows);
}
// Column blocks of a BN-wide tile (gate/up: BN / 2 h-columns per block).
template <int MODE, int BN>
LF_DEVICE int dense_gx(int ld) {
  return MODE == 2 ? ld / (BN / 2) : ld / BN;
}

// Writes bf16 NaN over the live rows of output tile (m0, bx): a 256-row
// form bound to a weight it cannot address (K >= 2^24).
template <int MODE, int BN>
LF_DEVICE void poison_tile(uint16_t *y, int ld, int M, int m0, int BM, int bx) {
  constexpr int cols = MODE == 2 ? BN / 2 : BN;
  const int rows = M - m0 < BM ? M - m0 : BM;
  for (int e = threadIdx.x; e < rows * cols; e += blockDim.x) {
    y[static_cast<uint64_t>(m0 + e / cols) * ld + bx * cols + e % cols] = 0x7FC0u;
  }
}

// ---------------------------------------------------------------------------
// W8A8 GEMM: xq [M, K] e4m3 with per-token scales (the quantizer's output) x
// weights with per-channel scales, y = bf16(acc * sa[m] * sw[n]). MODE 0:
// dense, 1: qkv (three weights, packed Q|K|V columns), 2: gate/up with the
// SwiGLU epilogue h = silu(g) * u.
//
// This form runs the direct-to-LDS main loop of w8a8_v3.h: BM x BN block of
// WGM x WGN waves, NS LDS stages, 1-D grid in the XCD-aware tile order
// (tile_of_block, GROUP row blocks per group). Block-local B slot s holds one 16-column weight tile; for
// gate/up, wave wn's kFN slots are kFN/2 gate tiles followed by the up tiles
// of the same columns, so the SwiGLU epilogue pairs accumulators inside a
// lane. Rows past the live M load a valid row (the last live one); their
// results are never stored.
// ---------------------------------------------------------------------------
template <class T, int GROUP, int MODE, bool THROUGH = false, class Gate = Open>
__device__ __forceinline__ int w8a8_tiled_kernel(uint8_t *smem, const int32_t *counts, const uint8_t *xq,
                                                 const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                                 uint16_t *y, int bid = -1, int capacity = 1 << 30,
                                                 const Gate &gate = Gate{}) {
  constexpr int BM = T::kWaveM * T::kWgm, BN = T::kWaveN * T::kWgn;
  const WeightHeader &h0 = header_of(w0);
  if (!dense_regions_ok<MODE>(w0, w1, w2)) return -1;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int M = live_rows(counts, capacity);
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = dense_ld<MODE>(w0, w1, w2);
  const int gx = dense_gx<MODE, BN>(ld);
  int bx, by;
  if (!w8a8v3::tile_of_block(bid < 0 ? static_cast<int>(blockIdx.x) : bid, gx, (M + BM - 1) / BM, GROUP,
                             bx, by)) {
    return -1;
  }
  const int m0 = by * BM;
  if (!gate(m0)) return -1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;

  // Weight tile of block slot s: region, tile index inside it, output column.
  auto slot = [&](int s, const uint8_t *&region, int &t, int &ocol) {
    if (MODE == 2) {
      const int sw = s / T::kFN, f = s % T::kFN;
      const bool up = f >= T::kFN / 2;
      const int col = bx * (BN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN / 2 : f);
      region = up ? w1 : w0;
      t = col >> 4;
      ocol = col;
    } else {
      t = bx * (BN / 16) + s;
      ocol = t * 16;
      region = w0;
      if (MODE == 1) {
        if (t >= tq + tk) {
          region = w2;
          t -= tq + tk;
        } else if (t >= tq) {
          region = w1;
          t -= tq;
        }
      }
    }
  };

  w8a8v3::Plan<T> plan;
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v3::a_load_row<T>(wave, q, lane);
    const int row = m0 + tr < M ? m0 + tr : M - 1;
    plan.a[q] = xq + static_cast<uint64_t>(row) * K + w8a8v3::a_load_chunk(tr, lane) * 16;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const int half = w8a8v3::b_load_half<T>(wave, q);
    const uint8_t *region;
    int t, ocol;
    slot(half >> 1, region, t, ocol);
    plan.b[q] = expert_tiles(region, 0) + static_cast<uint64_t>(t) * KT * kTileBytes +
                (half & 1) * 1024 + lane * 16;
  }
  f32x4 acc[T::kFM][T::kFN];
  w8a8v3::mainloop<T>(plan, KT, smem, acc);

  const float *ascale = reinterpret_cast<const float *>(xq + align256(static_cast<uint64_t>(M) * K));
  const int r = lane & 15;
  float swv[T::kFN];
  int ocol[T::kFN];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    int t;
    slot(wn * T::kFN + j, region, t, ocol[j]);
    swv[j] = expert_scales(region, 0)[t * 16 + r];
  }
  // Every scale this lane needs is loaded before the first store (the
  // stores may alias the scale arrays as far as the compiler knows, so a
  // load between stores would wait for them: one round trip per row).
  float sav[T::kFM][4];
#pragma unroll
  for (int i = 0; i < T::kFM; ++i)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int m = m0 + w8a8v3::acc_row<T>(wm, i, lane, rr);
      sav[i][rr] = ascale[m < M ? m : M - 1];
    }
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int m = m0 + w8a8v3::acc_row<T>(wm, i, lane, rr);
      if (m >= M) continue;
      const float sa = sav[i][rr];
      uint16_t *yrow = y + static_cast<uint64_t>(m) * ld;
      auto put = [&](int col, float v) {
        const uint16_t bits = static_cast<uint16_t>(f32_to_bf16(v));
        if constexpr (THROUGH) {
          __hip_atomic_store(yrow + col, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          yrow[col] = bits;
        }
      };
      if (MODE == 2) {
#pragma unroll
        for (int j = 0; j < T::kFN / 2; ++j) {
          const float gv = acc[i][j][rr] * sa * swv[j];
          const float uv = acc[i][j + T::kFN / 2][rr] * sa * swv[j + T::kFN / 2];
          put(ocol[j] + r, silu_mul(gv, uv));
        }
      } else {
#pragma unroll
        for (int j = 0; j < T::kFN; ++j) put(ocol[j] + r, acc[i][j][rr] * sa * swv[j]);
      }
    }
  }
  return by;
}

// ---------------------------------------------------------------------------
// Block-scaled W8A8: weights with 128 x 128 block scales (s[N/128][K/128]),
// activations quantized per 128-column group (the per-group quantizer's
// codes and scales), so both scales change with the k-tile:
//   y[m][n] = sum_kt (sa[m][kt] sw[n / 128][kt]) sum_{k in kt} qa[m][k] qw[n][k]
// in fp32, each k-tile's products folded into the running sum with its two
// scales (the main loop of w8a8_v3.h with a fold, as the block-scaled
// grouped GEMM does), no scale in the epilogue. The activation scales are
// stored k-tile-major (scales_t[kt][cap]: a 128-row tile's scales of one
// k-tile are 512 contiguous bytes) and arrive with each k-step's operands
// (one more LDS-direct load per wave, ScaleSide) in a window of NS slots,
// so K is not limited by LDS; the weight block scales are wave-uniform and
// read with scalar loads.
// ---------------------------------------------------------------------------
LF_DEVICE const float *uniform_f32(const float *p) {
  return reinterpret_cast<const float *>(w8a8v3::uniform_ptr(reinterpret_cast<const uint8_t *>(p)));
}

// Per-128-column-group quantizer of rows row0 .. row0 + rows - 1 (a chunk of
// a one-launch operation): the arithmetic of quantize_groups_wave (16 lanes
// per group, four groups per wave instruction, loads of eight quads in
// flight), codes in the row-major act-quant layout and the scale of (row,
// group g) at scales_t[g cap + row]. Wave gw of nw takes quads gw, gw + nw,
// ...; THROUGH: stores written through the XCD's L2 (phases.h).
template <bool THROUGH>
LF_DEVICE void quantize_group_rows(const uint16_t *x, int K, int row0, int rows, uint8_t *xq,
                                   float *scales_t, int cap, int gw, int nw) {
  const int lane = threadIdx.x & 63;
  const int per_row = K >> 7;
  const int groups = rows * per_row;
  const int quads = (groups + 3) >> 2;
  constexpr int kBatch = 8;
  for (int q0 = gw; q0 < quads; q0 += kBatch * nw) {
    uint4 v[kBatch];
    uint64_t base[kBatch];
    int sidx[kBatch];
    bool live[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int gid = 4 * (q0 + b * nw) + (lane >> 4);
      live[b] = gid < groups;
      const int r = live[b] ? gid / per_row : 0, kg = live[b] ? gid - r * per_row : 0;
      base[b] = static_cast<uint64_t>(row0 + r) * K + kg * 128 + (lane & 15) * 8;
      sidx[b] = kg * cap + row0 + r;
      v[b] = live[b] ? *reinterpret_cast<const uint4 *>(x + base[b]) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      float amax = bf16x8_amax(v[b], 0.0f);
      amax = fmaxf(amax, dpp_f32<0xB1>(amax));   // quad_perm [1, 0, 3, 2]
      amax = fmaxf(amax, dpp_f32<0x4E>(amax));   // quad_perm [2, 3, 0, 1]
      amax = fmaxf(amax, dpp_f32<0x141>(amax));  // row_half_mirror
      amax = fmaxf(amax, dpp_f32<0x140>(amax));  // row_mirror
      const bool zero = amax == 0.0f;
      const float ratio = zero ? 0.0f : 448.0f / amax;
      if (live[b]) {
        const uint2 e = bf16x8_encode(v[b], ratio, zero);
        store_codes8<THROUGH>(xq + base[b], e.x, e.y);
        if ((lane & 15) == 0) store_scale<THROUGH>(scales_t + sidx[b], zero ? 0.0f : amax / 448.0f);
      }
    }
  }
}

// Fold of one k-tile: acc += products x (sa[row][kt] x sw[block][kt]).
template <class T>
struct DenseBlockFold {
  static constexpr bool kActive = true;
  static constexpr int kBM = T::kWaveM * T::kWgm;
  const float *win;           // LDS [NS][kBM]: slot kt % NS holds k-tile kt's row scales
  int wm, lane;
  const float *sw[T::kFN];    // fragment j: [KT] scales of its 128-column block (wave-uniform)
  template <class A>
  LF_DEVICE void operator()(int kt, const A &step, A &acc, int) const {
    float swk[T::kFN];
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) swk[j] = sw[j][kt];
    const float *sa_k = win + (kt % T::kStages) * kBM;
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float sa = sa_k[w8a8v3::acc_row<T>(wm, i, lane, rr)];
#pragma unroll
        for (int j = 0; j < T::kFN; ++j) acc[i][j][rr] += step[i][j][rr] * (sa * swk[j]);
      }
    }
  }
};

// Side load of k-step kt: the tile's kBM activation scales of k-tile kt
// (scales_t row kt from the tile's first row) into window slot kt % NS,
// kBM / waves rows per wave (the first 16-byte lanes of one instruction).
template <class T>
struct ScaleSide {
  static constexpr int kIns = 1;
  static constexpr int kBM = T::kWaveM * T::kWgm;
  static constexpr int kLanes = kBM / T::kWaves / 4;
  static_assert(kLanes >= 1 && kLanes <= 64 && kBM % (4 * T::kWaves) == 0, "scale rows per wave");
  const uint8_t *base;  // scales_t + first row of the tile
  uint64_t stride;      // bytes per k-tile: cap * 4
  uint32_t win;         // LDS byte offset of the window
  LF_DEVICE void issue(int kt, int slot) const {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t part = static_cast<uint32_t>(wave) * kLanes * 16;
    if (lane < kLanes) {
      w8a8v3::dma16(w8a8v3::uniform_ptr(base + static_cast<uint64_t>(kt) * stride), part + lane * 16,
                    win + static_cast<uint32_t>(slot) * kBM * 4 + part);
    }
  }
};

// The block-scaled GEMM on one tile of the 128 x 128 form (4 waves, a block
// of T's shape): operand mapping, gate and THROUGH as w8a8_tiled_kernel; M
// live rows of a workspace sized for cap rows (xq [cap, K] codes, scales_t
// [K / 128][cap]); win: the block's window, T::kStages x BM floats of LDS.
template <class T, int GROUP, int MODE, bool THROUGH = false, class Gate = Open>
LF_DEVICE int w8a8_b128_gemm(uint8_t *smem, float *win, int M, const uint8_t *xq, const float *scales_t,
                             int cap, const uint8_t *w0, const uint8_t *w1, const uint8_t *w2, uint16_t *y,
                             int bid, const Gate &gate) {
  constexpr int BM = T::kWaveM * T::kWgm, BN = T::kWaveN * T::kWgn;
  const WeightHeader &h0 = header_of(w0);
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = dense_ld<MODE>(w0, w1, w2);
  const int gx = dense_gx<MODE, BN>(ld);
  int bx, by;
  if (!w8a8v3::tile_of_block(bid, gx, (M + BM - 1) / BM, GROUP, bx, by)) return -1;
  const int m0 = by * BM;
  if (!gate(m0)) return -1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;

  // Weight tile of block slot s: region, tile index inside it, output column
  // (the mapping of w8a8_tiled_kernel).
  auto slot = [&](int s, const uint8_t *&region, int &t, int &ocol) {
    if (MODE == 2) {
      const int sw = s / T::kFN, f = s % T::kFN;
      const bool up = f >= T::kFN / 2;
      const int col = bx * (BN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN / 2 : f);
      region = up ? w1 : w0;
      t = col >> 4;
      ocol = col;
    } else {
      t = bx * (BN / 16) + s;
      ocol = t * 16;
      region = w0;
      if (MODE == 1) {
        if (t >= tq + tk) {
          region = w2;
          t -= tq + tk;
        } else if (t >= tq) {
          region = w1;
          t -= tq;
        }
      }
    }
  };

  w8a8v3::Plan<T> plan;
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v3::a_load_row<T>(wave, q, lane);
    const int row = m0 + tr < M ? m0 + tr : M - 1;
    plan.a[q] = xq + static_cast<uint64_t>(row) * K + w8a8v3::a_load_chunk(tr, lane) * 16;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const int half = w8a8v3::b_load_half<T>(wave, q);
    const uint8_t *region;
    int t, ocol;
    slot(half >> 1, region, t, ocol);
    plan.b[q] = expert_tiles(region, 0) + static_cast<uint64_t>(t) * KT * kTileBytes +
                (half & 1) * 1024 + lane * 16;
  }
  DenseBlockFold<T> fold{win, wm, lane, {}};
  int ocol[T::kFN];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    int t;
    slot(wn * T::kFN + j, region, t, ocol[j]);
    // the 16-column tile t lies in 128-row block t / 8 of its region
    fold.sw[j] = uniform_f32(expert_scales(region, 0) + static_cast<uint64_t>(t >> 3) * KT);
  }
  const ScaleSide<T> side{w8a8v3::uniform_ptr(reinterpret_cast<const uint8_t *>(scales_t + m0)),
                          static_cast<uint64_t>(cap) * 4, w8a8v3::lds_offset_of(reinterpret_cast<uint8_t *>(win))};
  f32x4 acc[T::kFM][T::kFN];
  w8a8v3::mainloop<T, DenseBlockFold<T>, false, ScaleSide<T>>(plan, KT, smem, acc, fold, T::kFM, side);

  const int r = lane & 15;
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int m = m0 + w8a8v3::acc_row<T>(wm, i, lane, rr);
      if (m >= M) continue;
      uint16_t *yrow = y + static_cast<uint64_t>(m) * ld;
      auto put = [&](int col, float v) {
        const uint16_t bits = static_cast<uint16_t>(f32_to_bf16(v));
        if constexpr (THROUGH) {
          __hip_atomic_store(yrow + col, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          yrow[col] = bits;
        }
      };
      if (MODE == 2) {
#pragma unroll
        for (int j = 0; j < T::kFN / 2; ++j) put(ocol[j] + r, silu_mul(acc[i][j][rr], acc[i][j + T::kFN / 2][rr]));
      } else {
#pragma unroll
        for (int j = 0; j < T::kFN; ++j) put(ocol[j] + r, acc[i][j][rr]);
      }
    }
  }
  return by;
}

// ---------------------------------------------------------------------------
// W8A8 GEMM on the half-step main loop (w8a8_v4.h, 32 x 32 x 64 MFMA): BM x BN
// block of WGM x WGN waves, NS LDS stages, 1-D grid in the XCD-aware tile
// order. Operands and epilogues as w8a8_tiled_kernel. Block-local weight tile s
// (16 columns) maps to an output column through slot(); for gate/up, wave
// wn's 2 kFN tiles are kFN gate tiles followed by the up tiles of the same
// columns, so 32-column fragment j (gate) pairs with j + kFN / 2 (up).
// ---------------------------------------------------------------------------
template <class T, int GROUP, int MODE, bool THROUGH = false, class Gate = Open>
__device__ __forceinline__ int w8a8_v4_kernel(uint8_t *smem, const int32_t *counts, const uint8_t *xq,
                                              const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                              uint16_t *y, int bid = -1, int capacity = 1 << 30,
                                              const Gate &gate = Gate{}) {
  constexpr int BM = T::kBM, BN = T::kBN;
  const WeightHeader &h0 = header_of(w0);
  if (!dense_regions_ok<MODE>(w0, w1, w2)) return -1;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int M = live_rows(counts, capacity);
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = dense_ld<MODE>(w0, w1, w2);
  const int gx = dense_gx<MODE, BN>(ld);
  int bx, by;
  if (!w8a8v3::tile_of_block(bid < 0 ? static_cast<int>(blockIdx.x) : bid, gx, (M + BM - 1) / BM, GROUP,
                             bx, by)) {
    return -1;
  }
  const int m0 = by * BM;
  // 32-bit activation offsets need K < 2^24 (the geometry never picks this
  // form for wider K); a tile bound to such a weight anyway is filled with
  // NaN rather than left stale.
  if (K >= (1 << 24)) {
    poison_tile<MODE, BN>(y, ld, M, m0, BM, bx);
    return by;
  }
  if (!gate(m0)) return -1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;

  // Weight tile of block-local tile s: region, tile index inside it, output
  // column of its first column.
  auto slot = [&](int s, const uint8_t *&region, int &t, int &ocol) {
    if (MODE == 2) {
      const int sw = s / (2 * T::kFN), f = s % (2 * T::kFN);
      const bool up = f >= T::kFN;
      const int col = bx * (BN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN : f);
      region = up ? w1 : w0;
      t = col >> 4;
      ocol = col;
    } else {
      t = bx * (BN / 16) + s;
      ocol = t * 16;
      region = w0;
      if (MODE == 1) {
        if (t >= tq + tk) {
          region = w2;
          t -= tq + tk;
        } else if (t >= tq) {
          region = w1;
          t -= tq;
        }
      }
    }
  };

  // Row scales of the tile, one per thread of the first BM, loaded before
  // the main loop and parked in LDS after it for the epilogue.
  const float *ascale = reinterpret_cast<const float *>(xq + align256(static_cast<uint64_t>(M) * K));
  __shared__ float sa_tile[BM];
  float sa_mine = 0.0f;
  if (threadIdx.x < BM) {
    const int m = m0 + static_cast<int>(threadIdx.x);
    sa_mine = ascale[m < M ? m : M - 1];
  }
  // A offsets from the tile's first row: below 256 K < 2^32 for K < 2^24
  // (the launch geometry picks this form only then).
  w8a8v4::Plan<T> plan;
  plan.a_base = w8a8v3::uniform_ptr(xq + static_cast<uint64_t>(m0) * K);
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v4::a_load_row<T>(wave, q, lane);
    const int row = m0 + tr < M ? tr : M - 1 - m0;
    plan.a_off[q] = static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + w8a8v4::a_load_slot(tr, lane) * 32;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const uint8_t *region;
    int t, ocol;
    slot(w8a8v4::b_load_tile<T>(wave, q), region, t, ocol);
    plan.b_base[q] = w8a8v3::uniform_ptr(expert_tiles(region, 0) + static_cast<uint64_t>(t) * KT * kTileBytes);
  }
  plan.b_lane = lane * 16;
  w8a8v4::f32x16 acc[T::kFM][T::kFN];
  w8a8v4::mainloop<T>(plan, KT, smem, acc);

  if (threadIdx.x < BM) sa_tile[threadIdx.x] = sa_mine;
  const int c = lane & 31;
  float swv[T::kFN];
  int ocol[T::kFN];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    int t;
    slot((wn * T::kWaveN) / 16 + 2 * j + (c >> 4), region, t, ocol[j]);
    ocol[j] += c & 15;
    swv[j] = expert_scales(region, 0)[t * 16 + (c & 15)];
  }
  // The wave's output block is contiguous: rows m0 + wm kWaveM + [0, kWaveM),
  // columns from the first fragment's column (gate/up: kWaveN / 2 h-columns).
  // Staged one 32-row fragment row at a time (a whole 64-row wave tile with
  // the bank padding would not fit the 128 KiB ring for 128 columns).
  constexpr int kCols = MODE == 2 ? T::kWaveN / 2 : T::kWaveN;
  using Stage = w8a8v4::StageTile<uint16_t, 32, kCols>;
  static_assert(Stage::kBytes * T::kWaves <= T::kSmem, "staging fits the stage ring");
  const int col0 = __builtin_amdgcn_readfirstlane(ocol[0] - c);
  w8a8v4::epilogue_barrier();
  const Stage st{reinterpret_cast<uint16_t *>(smem + wave * Stage::kBytes)};
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = w8a8v4::acc_row<T>(0, lane, e);
      const float sa = sa_tile[wm * T::kWaveM + w8a8v4::acc_row<T>(i, lane, e)];
      if (MODE == 2) {
#pragma unroll
        for (int j = 0; j < T::kFN / 2; ++j) {
          const float gv = acc[i][j][e] * sa * swv[j];
          const float uv = acc[i][j + T::kFN / 2][e] * sa * swv[j + T::kFN / 2];
          st.put(row, ocol[j] - col0, static_cast<uint16_t>(f32_to_bf16(silu_mul(gv, uv))));
        }
      } else {
#pragma unroll
        for (int j = 0; j < T::kFN; ++j) {
          st.put(row, ocol[j] - col0, static_cast<uint16_t>(f32_to_bf16(acc[i][j][e] * sa * swv[j])));
        }
      }
    }
    const int mw = m0 + wm * T::kWaveM + 32 * i;
    st.template flush<THROUGH>(lane, [&](int row) -> uint16_t * {
      return mw + row < M ? y + static_cast<uint64_t>(mw + row) * ld + col0 : nullptr;
    });
  }
  return by;
}

// ---------------------------------------------------------------------------
// W8A8 GEMM on the four-wave 256-row loop (w8a8_v5.h, 16 x 16 x 128 MFMA
// with the weight fragment first; T: 256 x 256 or 256 x 128 tiles): 1-D grid
// in the XCD-aware tile order, operands as w8a8_tiled_kernel (block-local
// weight tile s = kFN wn + j is wave wn's fragment j; for gate/up, the first
// kFN / 2 fragments are gate tiles and the rest the up tiles of the same
// columns). Each lane holds one output row and four
// consecutive columns per accumulator, so the epilogue stages a wave's
// output through LDS with one 8-byte write per accumulator and stores whole
// 16-byte row chunks.
// ---------------------------------------------------------------------------
template <class T, int GROUP, int MODE, bool THROUGH = false, class Gate = Open>
__device__ __forceinline__ int w8a8_v5_kernel(uint8_t *smem, const int32_t *counts, const uint8_t *xq,
                                              const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                              uint16_t *y, int bid = -1, int capacity = 1 << 30,
                                              const Gate &gate = Gate{}) {
  constexpr int BM = 256, BN = T::kWaveN * T::kWgn;
  const WeightHeader &h0 = header_of(w0);
  if (!dense_regions_ok<MODE>(w0, w1, w2)) return -1;
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int M = live_rows(counts, capacity);
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = dense_ld<MODE>(w0, w1, w2);
  const int gx = dense_gx<MODE, BN>(ld);
  int bx, by;
  if (!w8a8v3::tile_of_block(bid < 0 ? static_cast<int>(blockIdx.x) : bid, gx, (M + BM - 1) / BM, GROUP,
                             bx, by)) {
    return -1;
  }
  const int m0 = by * BM;
  // 32-bit activation offsets need K < 2^24 (as in w8a8_v4_kernel)
  if (K >= (1 << 24)) {
    poison_tile<MODE, BN>(y, ld, M, m0, BM, bx);
    return by;
  }
  if (!gate(m0)) return -1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;

  // Weight tile of block-local tile s: region, tile index inside it, output
  // column of its first column.
  auto slot = [&](int s, const uint8_t *&region, int &t, int &ocol) {
    if (MODE == 2) {
      const int sw = s / T::kFN, f = s % T::kFN;
      const bool up = f >= T::kFN / 2;
      const int col = bx * (BN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN / 2 : f);
      region = up ? w1 : w0;
      t = col >> 4;
      ocol = col;
    } else {
      t = bx * (BN / 16) + s;
      ocol = t * 16;
      region = w0;
      if (MODE == 1) {
        if (t >= tq + tk) {
          region = w2;
          t -= tq + tk;
        } else if (t >= tq) {
          region = w1;
          t -= tq;
        }
      }
    }
  };

  // Row scales of the tile, one per thread, loaded before the main loop and
  // parked in LDS after it for the epilogue.
  const float *ascale = reinterpret_cast<const float *>(xq + align256(static_cast<uint64_t>(M) * K));
  __shared__ float sa_tile[BM];
  float sa_mine;
  {
    const int m = m0 + static_cast<int>(threadIdx.x);
    sa_mine = ascale[m < M ? m : M - 1];
  }
  // A offsets from the tile's first row: below 256 K + K < 2^32 for K <
  // 2^24 (the launch geometry picks this form only then).
  w8a8v5::Plan<T> plan;
  plan.a_base = w8a8v3::uniform_ptr(xq + static_cast<uint64_t>(m0) * K);
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v3::a_load_row<T>(wave, q, lane);
    const int row = m0 + tr < M ? tr : M - 1 - m0;
    plan.a_off[q] = static_cast<uint32_t>(row) * static_cast<uint32_t>(K) +
                    w8a8v3::a_load_chunk(tr, lane) * 16;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const int half = w8a8v3::b_load_half<T>(wave, q);
    const uint8_t *region;
    int t, ocol;
    slot(half >> 1, region, t, ocol);
    plan.b_base[q] = w8a8v3::uniform_ptr(expert_tiles(region, 0) +
                                         static_cast<uint64_t>(t) * KT * kTileBytes + (half & 1) * 1024);
  }
  plan.b_lane = lane * 16;
  f32x4 acc[T::kFM][T::kFN];
  w8a8v5::mainloop<T, true>(plan, KT, smem, acc);

  sa_tile[threadIdx.x] = sa_mine;
  // Column scales: four consecutive columns of each fragment per lane.
  float4 swv[T::kFN];
  int ocol[T::kFN];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    int t;
    slot(wn * T::kFN + j, region, t, ocol[j]);
    swv[j] = *reinterpret_cast<const float4 *>(expert_scales(region, 0) + t * 16 + 4 * (lane >> 4));
  }
  // A wave's output block is rows m0 + wm 128 + [0, 128) and kCols
  // consecutive columns from its first fragment's column (gate/up: 64
  // h-columns), staged kRows rows at a time.
  constexpr int kCols = MODE == 2 ? T::kWaveN / 2 : T::kWaveN;
  constexpr int kRows = kCols <= 64 ? 128 : 64;
  using Stage = w8a8v4::StageTile<uint16_t, kRows, kCols>;
  static_assert(Stage::kBytes * T::kWaves <= T::kSmem, "staging fits the stage ring");
  const int col0 = __builtin_amdgcn_readfirstlane(ocol[0]);
  w8a8v4::epilogue_barrier();
  const Stage st{reinterpret_cast<uint16_t *>(smem + wave * Stage::kBytes)};
  constexpr int kPassRows = kRows / 16;
#pragma unroll
  for (int p = 0; p < T::kFM / kPassRows; ++p) {
#pragma unroll
    for (int ii = 0; ii < kPassRows; ++ii) {
      const int i = p * kPassRows + ii;
      const int row = w8a8v5::acc_row(ii, lane);
      const float sa = sa_tile[wm * T::kWaveM + w8a8v5::acc_row(i, lane)];
      if (MODE == 2) {
#pragma unroll
        for (int j = 0; j < T::kFN / 2; ++j) {
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = acc[i][j][q] * sa * swv[j][q];
            const float uv = acc[i][j + T::kFN / 2][q] * sa * swv[j + T::kFN / 2][q];
            b[q] = f32_to_bf16(silu_mul(gv, uv));
          }
          st.put4(row, ocol[j] - col0 + 4 * (lane >> 4), b);
        }
      } else {
#pragma unroll
        for (int j = 0; j < T::kFN; ++j) {
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) b[q] = f32_to_bf16(acc[i][j][q] * sa * swv[j][q]);
          st.put4(row, ocol[j] - col0 + 4 * (lane >> 4), b);
        }
      }
    }
    const int mw = m0 + wm * T::kWaveM + kRows * p;
    st.template flush<THROUGH>(lane, [&](int row) -> uint16_t * {
      return mw + row < M ? y + static_cast<uint64_t>(mw + row) * ld + col0 : nullptr;
    });
  }
  return by;
}

// ---------------------------------------------------------------------------
// The W8A8 GEMM forms the launch geometry picks: tile height, block size and
// LDS of each, and its body.
// ---------------------------------------------------------------------------
template <class T, int GROUP>
struct FormT128 {  // 128 x 128 tiles, 4 waves, two blocks per CU
  static constexpr int kBM = T::kWaveM * T::kWgm, kBN = T::kWaveN * T::kWgn;
  static constexpr int kThreads = T::kThreads, kSmem = T::kSmem;
  // widest register-resident row of an in-launch quantizer (quantize_row_wave):
  // wider ones would cost this form its second wave per SIMD
  static constexpr int kQuantChunks = 8;
  template <int MODE, bool THROUGH = false, class Gate = Open>
  LF_DEVICE static int run(uint8_t *smem, const int32_t *counts, const uint8_t *xq, const uint8_t *w0,
                           const uint8_t *w1, const uint8_t *w2, uint16_t *y, int bid = -1,
                           int capacity = 1 << 30, const Gate &gate = Gate{}) {
    return w8a8_tiled_kernel<T, GROUP, MODE, THROUGH, Gate>(smem, counts, xq, w0, w1, w2, y, bid, capacity,
                                                           gate);
  }
};
template <class T, int GROUP>
struct FormW8 {  // 256 x 256 tiles on 8 waves, 4-stage half-step ring
  static constexpr int kBM = T::kBM, kBN = T::kBN;
  static constexpr int kThreads = T::kThreads, kSmem = T::kSmem;
  static constexpr int kQuantChunks = 32;
  template <int MODE, bool THROUGH = false, class Gate = Open>
  LF_DEVICE static int run(uint8_t *smem, const int32_t *counts, const uint8_t *xq, const uint8_t *w0,
                           const uint8_t *w1, const uint8_t *w2, uint16_t *y, int bid = -1,
                           int capacity = 1 << 30, const Gate &gate = Gate{}) {
    return w8a8_v4_kernel<T, GROUP, MODE, THROUGH, Gate>(smem, counts, xq, w0, w1, w2, y, bid, capacity,
                                                        gate);
  }
};
template <class T, int GROUP>
struct FormV5 {  // 256 x 256 / 256 x 128 tiles on 4 waves
  static constexpr int kBM = 256, kBN = T::kWaveN * T::kWgn;
  static constexpr int kThreads = T::kThreads, kSmem = T::kSmem;
  static constexpr int kQuantChunks = 32;
  template <int MODE, bool THROUGH = false, class Gate = Open>
  LF_DEVICE static int run(uint8_t *smem, const int32_t *counts, const uint8_t *xq, const uint8_t *w0,
                           const uint8_t *w1, const uint8_t *w2, uint16_t *y, int bid = -1,
                           int capacity = 1 << 30, const Gate &gate = Gate{}) {
    return w8a8_v5_kernel<T, GROUP, MODE, THROUGH, Gate>(smem, counts, xq, w0, w1, w2, y, bid, capacity,
                                                        gate);
  }
};

// Production tiles (lunaflux_fp8_launch_geometry picks): 256 x 256 on four
// waves (_t256) wherever a launch has at least one tile per CU; 256 x 256 on
// eight waves with the 4-stage half-step ring (_t256w8) from three quarters
// of a tile per CU up to that, where a CU runs a single tile and two waves
// per SIMD hide its load latency better (QKV at M = 2048, 192 tiles: 52.3
// against 57.5 us; from 512 tiles the four-wave form is 3-7 % faster);
// below, for QKV / dense, 256 x 128 on four waves (_t256x128, three stages)
// where that gives 128-256 tiles (o and down at M = 2048: 35.3 / 108.5
// against 38.9 / 121.0 us on 128 x 128; QKV at M = 1024 34.0 against 38.5;
// gate/up ran 10-18 % slower on it than on 256 x 256); 128 x 128 (4 waves,
// two blocks per CU) otherwise.
using GemmT256 = FormV5<w8a8v5::Tile, 4>;
using GemmT256x128 = FormV5<w8a8v5::TileN128, 4>;
using GemmT256w8 = FormW8<w8a8v4::Tile<256, 256, 4, 4, 2>, 4>;
using GemmT128 = FormT128<w8a8v3::Tile<128, 128, 2, 2, 2>, 4>;
// The same forms in the striped tile order (tile_of_block, group < 0), for
// the one-launch GatedMlp: every XCD works on the same group of row bands
// at a time, so the h quantizer and down steps find the first bands
// complete while gate/up's last tiles still run.
using GemmT256S = FormV5<w8a8v5::Tile, -4>;
using GemmT256x128S = FormV5<w8a8v5::TileN128, -4>;
using GemmT128S = FormT128<w8a8v3::Tile<128, 128, 2, 2, 2>, -4>;

// ---------------------------------------------------------------------------
// One launch per W8A8 operation. The plan binds each operation to one AOT
// entry point (kernels/launch_contract/types.mbt:16-27), and the operation's
// input is the bf16 activation, so the per-token quantizer runs inside the
// launch: the grid is kQuantBlocks quantizer blocks followed by the GEMM's
// blocks, and a GEMM tile starts its loads once every chunk (kChunkRows
// rows) of its row band is quantized (phases.h). Quantizer block q takes
// chunks q, q + kQuantBlocks, ...; each wave of it quantizes kChunkRows /
// waves rows of a chunk with the standalone quantizer's code (same codes
// and scales), its
// stores written through to memory, then the block counts the chunk into
// its band's counter.
// Workspace: the sync area (phases.h, one step of bands = ceil(max_tokens /
// BM) counters) followed by the quantized rows in the layout of
// lf_fp8_act_quant_rows' output (codes [M, K], fp32 scales at
// align256(M K)); bands = (gridDim.x - kQuantBlocks) / column blocks.
// ---------------------------------------------------------------------------
constexpr int kQuantBlocks = 256;
// 8-row chunks: at M = 2048 every quantizer block has one (16-row chunks left
// half of them idle and the other half ended 5-10 us into the launch).
constexpr int kChunkRows = 8;

LF_DEVICE int chunks_in_band(int M, int band, int BM) {
  const int rows = M - band * BM < BM ? M - band * BM : BM;
  return rows <= 0 ? 0 : (rows + kChunkRows - 1) / kChunkRows;
}

// The R = kChunkRows / waves rows of chunk c that this wave quantizes (at
// least one: an 8-wave block leaves waves past the chunk idle), in batches
// of register-resident rows (128 VGPRs of row data: 4 rows of <= 4096
// columns, 2 of <= 8192, 1 of <= 16384; F::kQuantChunks caps the row width
// of that form, wider rows take the two-pass form one at a time).
template <class F>
LF_DEVICE void quantize_chunk(const uint16_t *x, int K, int M, int c, uint8_t *xq, float *scales) {
  constexpr int kWaves = F::kThreads / 64;
  constexpr int R = kChunkRows / kWaves > 0 ? kChunkRows / kWaves : 1;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  if (wave * R >= kChunkRows) return;
  const int row0 = c * kChunkRows + wave * R;
  const int live = M - row0 < R ? M - row0 : R;
  if (live <= 0) return;
  auto batches = [&](auto chunks_tag, auto rows_tag) {
    constexpr int C = decltype(chunks_tag)::value, RB = decltype(rows_tag)::value;
#pragma unroll 1
    for (int i = 0; i < live; i += RB) {
      quantize_rows_wave_regs<C, RB, true>(x, K, row0 + i, live - i, xq, scales);
    }
  };
  using std::integral_constant;
  constexpr int RB8 = R < 4 ? R : 4, RB16 = R < 2 ? R : 2;
  if (K <= 4096) {
    batches(integral_constant<int, 8>{}, integral_constant<int, RB8>{});
  } else if (F::kQuantChunks >= 16 && K <= 8192) {
    batches(integral_constant<int, 16>{}, integral_constant<int, RB16>{});
  } else if (F::kQuantChunks >= 32 && K <= 16384) {
    batches(integral_constant<int, 32>{}, integral_constant<int, 1>{});
  } else {
#pragma unroll 1
    for (int i = 0; i < live; ++i) {
      const uint64_t off = static_cast<uint64_t>(row0 + i) * K;
      quantize_row_wave_2pass<true>(x + off, K, xq + off, scales + row0 + i);
    }
  }
}

template <class F, int MODE>
LF_DEVICE void w8a8_one_launch(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                               const uint8_t *w1, const uint8_t *w2, uint16_t *y, uint8_t *ws) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[F::kSmem];
  __shared__ phase::Flag flag;
  if (!dense_regions_ok<MODE>(w0, w1, w2)) return;
  const int K = static_cast<int>(header_of(w0).columns);
  const int gx = dense_gx<MODE, F::kBN>(dense_ld<MODE>(w0, w1, w2));
  const int blocks = static_cast<int>(gridDim.x) - kQuantBlocks;
  if (gx <= 0 || blocks <= 0 || blocks % gx != 0) return;  // not a grid of this entry's geometry
  const int bands = blocks / gx;
  const phase::Sync sync{reinterpret_cast<int *>(ws), bands};
  uint8_t *xq = ws + phase::sync_bytes(1, bands);
  const int cap = bands * F::kBM;
  const int M = live_rows(counts, cap);
  const int b = static_cast<int>(blockIdx.x);
  if (b < kQuantBlocks) {
    float *scales = reinterpret_cast<float *>(xq + align256(static_cast<uint64_t>(M) * K));
    const int chunks = (M + kChunkRows - 1) / kChunkRows;
    for (int c = b; c < chunks; c += kQuantBlocks) {
      quantize_chunk<F>(x, K, M, c, xq, scales);
      phase::signal(sync.band(0, c * kChunkRows / F::kBM));
    }
    return;
  }
  const auto gate = [&](int m0) {
    const int band = m0 / F::kBM;
    return phase::wait_for(sync, sync.band(0, band), chunks_in_band(M, band, F::kBM), flag);
  };
  F::template run<MODE>(smem, counts, xq, w0, w1, w2, y, b - kQuantBlocks, cap, gate);
  phase::finish(sync, blocks, 1, flag);
}

// ---------------------------------------------------------------------------
// Block-scaled W8A8 operations as one launch each (_b128 entries): the grid
// is kQuantBlocks per-group quantizer blocks followed by the GEMM's
// 128 x 128 tiles (4 waves), each tile starting once every chunk of its row
// band is quantized, as in w8a8_one_launch. Workspace: the sync area (one
// step of bands counters), codes [cap, K] (cap = bands x 128), then the
// group scales k-tile-major, [K / 128][cap] fp32 (B128Rows).
// ---------------------------------------------------------------------------
using B128Tile = w8a8v3::Tile<128, 128, 2, 2, 2>;
constexpr int kB128BM = 128;

struct B128Rows {
  uint8_t *codes;
  float *scales_t;
  uint64_t bytes;
};
LF_DEVICE B128Rows b128_rows(uint8_t *at, int cap, int K) {
  const uint64_t codes = align256(static_cast<uint64_t>(cap) * K);
  const uint64_t scales = align256(static_cast<uint64_t>(K >> 7) * cap * 4);
  return B128Rows{at, reinterpret_cast<float *>(at + codes), codes + scales};
}

// Quantizer step: block b (of kQuantBlocks) quantizes chunks b, b +
// kQuantBlocks, ... of kChunkRows rows (its 4 waves splitting each chunk's
// groups) and counts each into its band's counter of step `step`.
// BM: the GEMM's band height (the counter a chunk counts into).
template <int BM = kB128BM>
LF_DEVICE void b128_quantize(const uint16_t *x, int K, int M, const B128Rows &rows, int cap, int b,
                             const phase::Sync &sync, int step) {
  const int chunks = (M + kChunkRows - 1) / kChunkRows;
  const int wave = static_cast<int>(threadIdx.x) >> 6, nw = static_cast<int>(blockDim.x) >> 6;
  for (int c = b; c < chunks; c += kQuantBlocks) {
    const int row0 = c * kChunkRows;
    const int n = M - row0 < kChunkRows ? M - row0 : kChunkRows;
    quantize_group_rows<true>(x, K, row0, n, rows.codes, rows.scales_t, cap, wave, nw);
    phase::signal(sync.band(step, row0 / BM));
  }
}

template <int MODE>
LF_DEVICE void w8a8_b128_one_launch(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                                    const uint8_t *w1, const uint8_t *w2, uint16_t *y, uint8_t *ws) {
  using T = B128Tile;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::kSmem];
  __shared__ __attribute__((aligned(16))) float win[T::kStages * kB128BM];
  __shared__ phase::Flag flag;
  if (!dense_regions_ok<MODE, kScaleBlock128>(w0, w1, w2)) return;
  const int K = static_cast<int>(header_of(w0).columns);
  const int gx = dense_gx<MODE, 128>(dense_ld<MODE>(w0, w1, w2));
  const int blocks = static_cast<int>(gridDim.x) - kQuantBlocks;
  if (gx <= 0 || blocks <= 0 || blocks % gx != 0 || blockDim.x != T::kThreads) return;
  const int bands = blocks / gx;
  const phase::Sync sync{reinterpret_cast<int *>(ws), bands};
  const int cap = bands * kB128BM;
  const B128Rows rows = b128_rows(ws + phase::sync_bytes(1, bands), cap, K);
  const int M = live_rows(counts, cap);
  const int b = static_cast<int>(blockIdx.x);
  if (b < kQuantBlocks) {
    b128_quantize(x, K, M, rows, cap, b, sync, 0);
    return;
  }
  const auto gate = [&](int m0) {
    const int band = m0 / kB128BM;
    return phase::wait_for(sync, sync.band(0, band), chunks_in_band(M, band, kB128BM), flag);
  };
  w8a8_b128_gemm<T, 4, MODE>(smem, win, M, rows.codes, rows.scales_t, cap, w0, w1, w2, y, b - kQuantBlocks,
                             gate);
  phase::finish(sync, blocks, 1, flag);
}

// ---------------------------------------------------------------------------
// Block-scaled W8A8 on 256 x 256 tiles (the eight-wave half-step loop of
// w8a8_v4.h with swapped operands, as the block-scaled MoE GEMMs), which
// the launch geometry picks for profiles of at least 192 such tiles (fewer:
// the 128 x 128 form above keeps more CUs busy). The accumulators hold
// acc / sigma_kt with sigma_kt = a[row][kt] w[block][kt] (each scale
// sequence carries its last nonzero value forward, carry_ratio: a zero scale
// belongs only to an all-zero group, whose products are zero); before
// k-tile kt's first MFMA into a column fragment they are multiplied by
// sigma_{kt-1} / sigma_kt, and the epilogue multiplies by the last sigma.
// No table of all k-tiles fits beside the 128 KiB stage ring at these K
// (32-112 k-tiles), so each stage also side-loads its k-tile's activation
// scales of the tile's 256 rows into a two-slot LDS window, and the weight
// scales are scalar loads.
// ---------------------------------------------------------------------------
using B128V4Tile = w8a8v4::Tile<256, 256, 4, 4, 2>;
// 256 x 128 tiles: eight waves of 32 x 128 (each wave's columns still one
// 128-column block), for launches with too few 256 x 256 tiles
using B128V4TileN128 = w8a8v4::Tile<256, 128, 4, 8, 1>;
constexpr int kB128V4BM = 256;

// Side loads (w8a8v4 mainloop SIDE): stage s loads the 256 row scales of
// k-tile s / 2 (1 KiB of scales_t[kt][m0 ..]) into window slot (s / 2) & 1;
// both stages of a k-tile load the same bytes, so every stage has one load
// per wave and the waits stay uniform. Wave w loads rows 64 (w % 4) .. + 63,
// one dword per lane (waves w and w + 4 write the same bytes: a load with
// only some lanes active, a branch inside the half-step, cost the loop 70-190
// spilled registers). Slot reuse: k-tile kt + 2's first load is issued after
// the block barrier of half-step 2 kt + 1, when every wave has read k-tile
// kt's slot (at the start of half-step 2 kt); the second load of a k-tile
// rewrites its slot with the same bytes.
template <class T>
struct B128V4Side {
  static constexpr int kIns = 1;
  const uint8_t *base;  // scales_t + m0 (wave-uniform)
  uint64_t stride;      // bytes per k-tile: cap * 4
  uint32_t win;         // LDS byte offset of the window [2][kBM] fp32
  LF_DEVICE void issue(int s, int) const {
    static_assert(T::kBM == 256 && T::kWaves == 8, "four waves cover the 256 rows");
    const int lane = threadIdx.x & 63, part = (static_cast<int>(threadIdx.x) >> 6) & 3;
    const int kt = s >> 1;
    w8a8v3::dma4(w8a8v3::uniform_ptr(base + static_cast<uint64_t>(kt) * stride),
                 static_cast<uint32_t>(64 * part + lane) * 4,
                 win + static_cast<uint32_t>(kt & 1) * T::kBM * 4 + static_cast<uint32_t>(part) * 256);
  }
};

// Rescale (w8a8v4 mainloop RESCALE, swapped layout: lane l holds row
// row0 + 32 i of fragment i). Part 1: the up fragments of gate/up (column
// fragments kFN / 2 ..), whose weight block scales are the up weight's.
// The loop runs on a copy of the functor, so after the last k-tile's
// begin() the final sigma factors go to LDS (last: the tile's 256 row
// scales, then two per wave) for the epilogue.
template <class T, int MODE>
struct B128V4Rescale {
  static constexpr int kParts = MODE == 2 ? 2 : 1;
  typedef const __attribute__((address_space(3))) float *lds_ptr;
  typedef __attribute__((address_space(3))) float *lds_wptr;
  lds_ptr win;                 // [2][kBM] row scales (B128V4Side)
  lds_wptr last;               // [kBM + 2 kWaves]: last nonzero row / block scales
  int row0;                    // the lane's row of fragment 0 in the tile
  int KT;
  const float *sw[kParts];     // this wave's block scales [KT] per part (wave-uniform)
  float prev_a[T::kFM];        // last nonzero row scale so far (1 before any)
  float prev_w[kParts];
  float m[kParts][T::kFM];     // this k-tile's multipliers
  LF_DEVICE void begin(int kt) {
    float rw[kParts];
#pragma unroll
    for (int p = 0; p < kParts; ++p) rw[p] = carry_ratio(sload(sw[p], kt), prev_w[p]);
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
      const float ra = carry_ratio(win[(kt & 1) * T::kBM + row0 + 32 * i], prev_a[i]);
#pragma unroll
      for (int p = 0; p < kParts; ++p) m[p][i] = kt == 0 ? 1.0f : ra * rw[p];
    }
    if (kt == KT - 1) {
      // (lanes l and l + 32 hold the same rows: the same values)
#pragma unroll
      for (int i = 0; i < T::kFM; ++i) last[row0 + 32 * i] = prev_a[i];
      const int wave = threadIdx.x >> 6;
#pragma unroll
      for (int p = 0; p < kParts; ++p) last[T::kBM + 2 * wave + p] = prev_w[p];
    }
  }
  template <class A>
  LF_DEVICE void apply(int o, A &acc) {
    const int p = kParts == 2 && o >= T::kFN / 2 ? 1 : 0;
#pragma unroll
    for (int i = 0; i < T::kFM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][o][e] *= m[p][i];
  }
};

// The GEMM on one 256 x 256 tile of M live rows of a workspace sized for
// cap rows (codes [cap, K], scales_t [K / 128][cap]); operand mapping and
// gate as w8a8_b128_gemm; win: the block's LDS window (2 x 256 floats), then
// kBM + 2 kWaves floats for the final scales.
template <class T, int GROUP, int MODE, bool THROUGH = false, class Gate = Open>
LF_DEVICE int w8a8_b128_v4_gemm(uint8_t *smem, float *win, int M, const uint8_t *xq, const float *scales_t,
                                int cap, const uint8_t *w0, const uint8_t *w1, const uint8_t *w2, uint16_t *y,
                                int bid, const Gate &gate) {
  constexpr int BM = T::kBM, BN = T::kBN;
  static_assert(T::kWaveN == 128 && BM == kB128V4BM, "a wave's columns are one 128-column block");
  const WeightHeader &h0 = header_of(w0);
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int tq = static_cast<int>(h0.rows) >> 4;
  const int tk = MODE == 1 ? static_cast<int>(header_of(w1).rows) >> 4 : 0;
  const int ld = dense_ld<MODE>(w0, w1, w2);
  const int gx = dense_gx<MODE, BN>(ld);
  int bx, by;
  if (!w8a8v3::tile_of_block(bid, gx, (M + BM - 1) / BM, GROUP, bx, by)) return -1;
  const int m0 = by * BM;
  // 32-bit activation offsets (below 256 K) need K < 2^24
  if (K >= (1 << 24)) {
    poison_tile<MODE, BN>(y, ld, M, m0, BM, bx);
    return by;
  }
  if (!gate(m0)) return -1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;

  // Weight tile of block-local tile s (the mapping of w8a8_v4_kernel).
  auto slot = [&](int s, const uint8_t *&region, int &t, int &ocol) {
    if (MODE == 2) {
      const int sw = s / (2 * T::kFN), f = s % (2 * T::kFN);
      const bool up = f >= T::kFN;
      const int col = bx * (BN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN : f);
      region = up ? w1 : w0;
      t = col >> 4;
      ocol = col;
    } else {
      t = bx * (BN / 16) + s;
      ocol = t * 16;
      region = w0;
      if (MODE == 1) {
        if (t >= tq + tk) {
          region = w2;
          t -= tq + tk;
        } else if (t >= tq) {
          region = w1;
          t -= tq;
        }
      }
    }
  };

  w8a8v4::Plan<T> plan;
  plan.a_base = w8a8v3::uniform_ptr(xq + static_cast<uint64_t>(m0) * K);
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v4::a_load_row<T>(wave, q, lane);
    const int row = m0 + tr < M ? tr : M - 1 - m0;
    plan.a_off[q] = static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + w8a8v4::a_load_slot(tr, lane) * 32;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const uint8_t *region;
    int t, ocol;
    slot(w8a8v4::b_load_tile<T>(wave, q), region, t, ocol);
    plan.b_base[q] = w8a8v3::uniform_ptr(expert_tiles(region, 0) + static_cast<uint64_t>(t) * KT * kTileBytes);
  }
  plan.b_lane = lane * 16;

  // This wave's 128-column block: (gate/up) its 64 gate and 64 up columns
  // lie in one 128-row block of each weight; (dense, QKV) its 128 columns
  // are one block of one region (every QKV width is a multiple of 128).
  typedef const __attribute__((address_space(3))) float *lds_ptr;
  typedef __attribute__((address_space(3))) float *lds_wptr;
  float *last = win + 2 * BM;
  B128V4Rescale<T, MODE> rs;
  rs.win = (lds_ptr)(win);
  rs.last = (lds_wptr)(last);
  rs.row0 = wm * T::kWaveM + (lane & 31);
  rs.KT = KT;
#pragma unroll
  for (int p = 0; p < B128V4Rescale<T, MODE>::kParts; ++p) {
    const uint8_t *region;
    int t, ocol;
    slot(wn * (T::kWaveN / 16) + p * T::kFN, region, t, ocol);
    rs.sw[p] = reinterpret_cast<const float *>(w8a8v3::uniform_ptr(
        reinterpret_cast<const uint8_t *>(expert_scales(region, 0) + static_cast<uint64_t>(t >> 3) * KT)));
    rs.prev_w[p] = 1.0f;
  }
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) rs.prev_a[i] = 1.0f;
  const B128V4Side<T> side{w8a8v3::uniform_ptr(reinterpret_cast<const uint8_t *>(scales_t + m0)),
                           static_cast<uint64_t>(cap) * 4,
                           w8a8v3::lds_offset_of(reinterpret_cast<uint8_t *>(win))};
  w8a8v4::f32x16 acc[T::kFM][T::kFN];
  w8a8v4::mainloop<T, false, B128V4Rescale<T, MODE>, true, B128V4Side<T>>(plan, KT, smem, acc, T::kFM, rs,
                                                                         true, side);
  // the final sigma factors (this lane wrote its rows' and its wave's)
  float sa_last[T::kFM], sw_last[B128V4Rescale<T, MODE>::kParts];
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) sa_last[i] = last[rs.row0 + 32 * i];
#pragma unroll
  for (int p = 0; p < B128V4Rescale<T, MODE>::kParts; ++p) sw_last[p] = last[BM + 2 * wave + p];

  // Epilogue (swapped layout: element 4 g + q of fragment j is column
  // 32 j + 8 g + 4 (lane / 32) + q): times the last sigma, staged through
  // LDS one 32-row fragment at a time in 16-byte row chunks.
  const int rl = lane & 31, c4 = 4 * (lane >> 5);
  constexpr int kCols = MODE == 2 ? T::kWaveN / 2 : T::kWaveN;
  using Stage = w8a8v4::StageTile<uint16_t, 32, kCols>;
  static_assert(Stage::kBytes * T::kWaves <= T::kSmem, "staging fits the stage ring");
  int col0;
  {
    const uint8_t *region;
    int t;
    slot(wn * (T::kWaveN / 16), region, t, col0);
  }
  col0 = __builtin_amdgcn_readfirstlane(col0);
  w8a8v4::epilogue_barrier();
  const Stage st{reinterpret_cast<uint16_t *>(smem + wave * Stage::kBytes)};
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) {
    const float sa = sa_last[i];
    if constexpr (MODE == 2) {
#pragma unroll
      for (int j = 0; j < T::kFN / 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = acc[i][j][4 * g + q] * sa * sw_last[0];
            const float uv = acc[i][j + T::kFN / 2][4 * g + q] * sa * sw_last[B128V4Rescale<T, MODE>::kParts - 1];
            b[q] = f32_to_bf16(silu_mul(gv, uv));
          }
          st.put4(rl, 32 * j + 8 * g + c4, b);
        }
    } else {
#pragma unroll
      for (int j = 0; j < T::kFN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) b[q] = f32_to_bf16(acc[i][j][4 * g + q] * sa * sw_last[0]);
          st.put4(rl, 32 * j + 8 * g + c4, b);
        }
    }
    const int mw = m0 + wm * T::kWaveM + 32 * i;
    st.template flush<THROUGH>(lane, [&](int row) -> uint16_t * {
      return mw + row < M ? y + static_cast<uint64_t>(mw + row) * ld + col0 : nullptr;
    });
  }
  return by;
}

// The block-scaled operations in one launch on the 256 x 256 (or 256 x 128)
// form: as w8a8_b128_one_launch with 256-row bands (cap = bands x 256).
template <class T, int MODE>
LF_DEVICE void w8a8_b128_v4_one_launch(const int32_t *counts, const uint16_t *x, const uint8_t *w0,
                                       const uint8_t *w1, const uint8_t *w2, uint16_t *y, uint8_t *ws) {
  constexpr int BM = kB128V4BM;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::kSmem];
  __shared__ __attribute__((aligned(16))) float win[2 * BM + BM + 2 * T::kWaves];
  __shared__ phase::Flag flag;
  if (!dense_regions_ok<MODE, kScaleBlock128>(w0, w1, w2)) return;
  const int K = static_cast<int>(header_of(w0).columns);
  const int gx = dense_gx<MODE, T::kBN>(dense_ld<MODE>(w0, w1, w2));
  const int blocks = static_cast<int>(gridDim.x) - kQuantBlocks;
  if (gx <= 0 || blocks <= 0 || blocks % gx != 0 || blockDim.x != T::kThreads) return;
  const int bands = blocks / gx;
  const phase::Sync sync{reinterpret_cast<int *>(ws), bands};
  const int cap = bands * BM;
  const B128Rows rows = b128_rows(ws + phase::sync_bytes(1, bands), cap, K);
  const int M = live_rows(counts, cap);
  const int b = static_cast<int>(blockIdx.x);
  if (b < kQuantBlocks) {
    b128_quantize<BM>(x, K, M, rows, cap, b, sync, 0);
    return;
  }
  const auto gate = [&](int m0) {
    const int band = m0 / BM;
    return phase::wait_for(sync, sync.band(0, band), chunks_in_band(M, band, BM), flag);
  };
  w8a8_b128_v4_gemm<T, 4, MODE>(smem, win, M, rows.codes, rows.scales_t, cap, w0, w1, w2, y,
                                b - kQuantBlocks, gate);
  phase::finish(sync, blocks, 1, flag);
}

// Block-scaled tile forms of the one-launch GatedMlp: 0 = 128 x 128 (4
// waves), 2 = 256 x 256 (8 waves). (The 256 x 128 form of the standalone
// entries is not built here: in this kernel its gate/up step returned
// nondeterministic values in a few accumulator elements of one column
// fragment, different rows on every launch, with the cause not found; the
// standalone 256 x 128 entries measure bit-identical to 256 x 256.)
template <int FORM>
struct B128Form {
  static_assert(FORM == 0 || FORM == 2, "GatedMlp tile forms");
  using T = std::conditional_t<FORM == 2, B128V4Tile, std::conditional_t<FORM == 1, B128V4TileN128, B128Tile>>;
  static constexpr int kBM = FORM ? kB128V4BM : kB128BM, kBN = FORM == 2 ? 256 : 128;
  // LDS scale window: (256-row forms) two k-tile slots, then the final
  // scales; (128 x 128) one slot per stage
  static constexpr int kWin = FORM ? 3 * kBM + 2 * T::kWaves : T::kStages * kBM;
};

template <int FORM, int MODE, bool THROUGH, class Gate>
LF_DEVICE int w8a8_b128_form_gemm(uint8_t *smem, float *win, int M, const B128Rows &rows, int cap,
                                  const uint8_t *w0, const uint8_t *w1, uint16_t *out, int bid, const Gate &gate) {
  if constexpr (FORM != 0) {
    return w8a8_b128_v4_gemm<typename B128Form<FORM>::T, 4, MODE, THROUGH>(smem, win, M, rows.codes, rows.scales_t,
                                                                          cap, w0, w1, w1, out, bid, gate);
  } else {
    return w8a8_b128_gemm<B128Tile, 4, MODE, THROUGH>(smem, win, M, rows.codes, rows.scales_t, cap, w0, w1, w1,
                                                      out, bid, gate);
  }
}

// The block-scaled GatedMlp in one launch: x -> group quantizer -> gate/up
// + SwiGLU -> h (bf16) -> group quantizer -> down, four counted steps as in
// w8a8_gated_mlp, both GEMMs on one tile form (B128Form; the 256-row forms
// run 512-thread blocks in every step). Workspace: sync area (three steps
// of bands counters), B128Rows of x (K = H), h [cap, I] bf16, B128Rows of h
// (K = I).
template <int FORM>
LF_DEVICE void w8a8_b128_gated_mlp(const int32_t *counts, const uint16_t *x, const uint8_t *wg,
                                   const uint8_t *wu, const uint8_t *wd, uint16_t *y, uint8_t *ws) {
  using F = B128Form<FORM>;
  using T = typename F::T;
  constexpr int BM = F::kBM;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::kSmem];
  __shared__ __attribute__((aligned(16))) float win[F::kWin];
  __shared__ phase::Flag flag;
  if (!dense_regions_ok<2, kScaleBlock128>(wg, wu, wu) || !dense_regions_ok<0, kScaleBlock128>(wd, wd, wd)) {
    return;
  }
  const int H = static_cast<int>(header_of(wg).columns), I = static_cast<int>(header_of(wg).rows);
  if (static_cast<int>(header_of(wd).columns) != I || static_cast<int>(header_of(wd).rows) != H) return;
  int gx1 = dense_gx<2, F::kBN>(I), gx2 = dense_gx<0, F::kBN>(H);
  // (opaque to the optimizer: a range for H or I derived from the checks
  // below reshapes the 256 x 256 main loop's prologue and tail, whose
  // schedule then needs more than its 256 registers)
  asm("" : "+s"(gx1), "+s"(gx2));
  const int blocks = static_cast<int>(gridDim.x) - 2 * kQuantBlocks;
  if (gx1 <= 0 || gx2 <= 0 || blocks <= 0 || blocks % (gx1 + gx2) != 0 || blockDim.x != T::kThreads) return;
  const int bands = blocks / (gx1 + gx2);
  const phase::Sync sync{reinterpret_cast<int *>(ws), bands};
  const int cap = bands * BM;
  const B128Rows xr = b128_rows(ws + phase::sync_bytes(3, bands), cap, H);
  uint16_t *h = reinterpret_cast<uint16_t *>(xr.codes + xr.bytes);
  const B128Rows hr = b128_rows(reinterpret_cast<uint8_t *>(h) + align256(static_cast<uint64_t>(cap) * I * 2),
                                cap, I);
  const int M = live_rows(counts, cap);
  int b = static_cast<int>(blockIdx.x);
  if (b < kQuantBlocks) {  // step 0: x -> codes and group scales
    b128_quantize<BM>(x, H, M, xr, cap, b, sync, 0);
    return;
  }
  b -= kQuantBlocks;
  if (b < gx1 * bands) {  // step 1: gate/up + SwiGLU -> h
    const auto gate = [&](int m0) {
      const int band = m0 / BM;
      return phase::wait_for(sync, sync.band(0, band), chunks_in_band(M, band, BM), flag);
    };
    const int band = w8a8_b128_form_gemm<FORM, 2, true>(smem, win, M, xr, cap, wg, wu, h, b, gate);
    if (band >= 0) phase::signal(sync.band(1, band));
    return;
  }
  b -= gx1 * bands;
  if (b < kQuantBlocks) {  // step 2: h -> codes and group scales
    const int chunks = (M + kChunkRows - 1) / kChunkRows;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    for (int c = b; c < chunks; c += kQuantBlocks) {
      const int row0 = c * kChunkRows, band = row0 / BM;
      if (!phase::wait_for(sync, sync.band(1, band), gx1, flag)) return;
      const int n = M - row0 < kChunkRows ? M - row0 : kChunkRows;
      quantize_group_rows<true>(h, I, row0, n, hr.codes, hr.scales_t, cap, wave, T::kWaves);
      phase::signal(sync.band(2, band));
    }
    return;
  }
  b -= kQuantBlocks;
  const auto gate = [&](int m0) {  // step 3: down
    const int band = m0 / BM;
    return phase::wait_for(sync, sync.band(2, band), chunks_in_band(M, band, BM), flag);
  };
  w8a8_b128_form_gemm<FORM, 0, false>(smem, win, M, hr, cap, wd, wd, y, b, gate);
  phase::finish(sync, gx2 * bands, 3, flag);
}

// ---------------------------------------------------------------------------
// W8A8 GatedMlp in one launch (model/plan/plan.mbt:47-59;
// kernels/reference/mlp.mbt:4-39): x -> xq (per token) -> gate/up + SwiGLU ->
// h (bf16) -> hq (per token) -> down -> y, the same arithmetic as the
// act-quant, gate/up, act-quant and dense launches, as four steps of one
// grid: [kQuantBlocks x quantizer][gate/up tiles][kQuantBlocks h quantizer]
// [down tiles]. Gate/up tiles wait for their band's x chunks and write h
// through to memory; an h-quantizer chunk waits for every gate/up tile of its
// band; down tiles wait for their band's h chunks. Both GEMMs use the same
// band height and block size (GU::kBM, kThreads).
// Workspace: sync area (three steps of bands counters), xq for cap = bands
// BM rows (act-quant layout, K = H), h bf16 [cap, I], hq (act-quant layout,
// K = I); bands = (gridDim.x - 2 kQuantBlocks) / (gate/up + down column
// blocks).
// ---------------------------------------------------------------------------
template <class GU, class DN>
LF_DEVICE void w8a8_gated_mlp(const int32_t *counts, const uint16_t *x, const uint8_t *wg,
                              const uint8_t *wu, const uint8_t *wd, uint16_t *y, uint8_t *ws) {
  static_assert(GU::kBM == DN::kBM && GU::kThreads == DN::kThreads, "one band height, one block size");
  constexpr int BM = GU::kBM;
  constexpr int kSmem = GU::kSmem > DN::kSmem ? GU::kSmem : DN::kSmem;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmem];
  __shared__ phase::Flag flag;
  if (!dense_regions_ok<2>(wg, wu, wu) || !dense_regions_ok<0>(wd, wd, wd)) return;
  const int H = static_cast<int>(header_of(wg).columns), I = static_cast<int>(header_of(wg).rows);
  if (static_cast<int>(header_of(wd).columns) != I || static_cast<int>(header_of(wd).rows) != H) return;
  const int gx1 = dense_gx<2, GU::kBN>(I), gx2 = dense_gx<0, DN::kBN>(H);
  const int blocks = static_cast<int>(gridDim.x) - 2 * kQuantBlocks;
  if (gx1 <= 0 || gx2 <= 0 || blocks <= 0 || blocks % (gx1 + gx2) != 0) return;
  const int bands = blocks / (gx1 + gx2);
  const phase::Sync sync{reinterpret_cast<int *>(ws), bands};
  const int cap = bands * BM;
  const uint64_t xq_bytes = align256(static_cast<uint64_t>(cap) * H) + align256(static_cast<uint64_t>(cap) * 4);
  const uint64_t h_bytes = align256(static_cast<uint64_t>(cap) * I * 2);
  uint8_t *xq = ws + phase::sync_bytes(3, bands);
  uint16_t *h = reinterpret_cast<uint16_t *>(xq + xq_bytes);
  uint8_t *hq = xq + xq_bytes + h_bytes;
  const int M = live_rows(counts, cap);
  const int chunks = (M + kChunkRows - 1) / kChunkRows;
  int b = static_cast<int>(blockIdx.x);
  if (b < kQuantBlocks) {  // step 0: x -> xq
    float *scales = reinterpret_cast<float *>(xq + align256(static_cast<uint64_t>(M) * H));
    for (int c = b; c < chunks; c += kQuantBlocks) {
      quantize_chunk<GU>(x, H, M, c, xq, scales);
      phase::signal(sync.band(0, c * kChunkRows / BM));
    }
    return;
  }
  b -= kQuantBlocks;
  if (b < gx1 * bands) {  // step 1: gate/up + SwiGLU -> h
    const auto gate = [&](int m0) {
      const int band = m0 / BM;
      return phase::wait_for(sync, sync.band(0, band), chunks_in_band(M, band, BM), flag);
    };
    const int band = GU::template run<2, true>(smem, counts, xq, wg, wu, wu, h, b, cap, gate);
    if (band >= 0) phase::signal(sync.band(1, band));
    return;
  }
  b -= gx1 * bands;
  if (b < kQuantBlocks) {  // step 2: h -> hq
    float *scales = reinterpret_cast<float *>(hq + align256(static_cast<uint64_t>(M) * I));
    for (int c = b; c < chunks; c += kQuantBlocks) {
      const int band = c * kChunkRows / BM;
      if (!phase::wait_for(sync, sync.band(1, band), gx1, flag)) return;
      quantize_chunk<GU>(h, I, M, c, hq, scales);
      phase::signal(sync.band(2, band));
    }
    return;
  }
  b -= kQuantBlocks;
  const auto gate = [&](int m0) {  // step 3: down
    const int band = m0 / BM;
    return phase::wait_for(sync, sync.band(2, band), chunks_in_band(M, band, BM), flag);
  };
  DN::template run<0>(smem, counts, hq, wd, wd, wd, y, b, cap, gate);
  phase::finish(sync, gx2 * bands, 3, flag);
}

}  // namespace

extern "C" {

// GEMM alone over rows already quantized (lf_fp8_act_quant_rows or the fused
// RmsNorm quantizer): (counts, xq, w..., y). One launch with the quantizer
// (_aq): (counts, x, w..., y, ws).
#define LF_W8A8_ENTRIES(NAME, FORM)                                                             \
  __global__ __launch_bounds__(FORM::kThreads) void lf_fp8_w8a8_dense_##NAME(                  \
      const int32_t *counts, const uint8_t *xq, const uint8_t *w, uint16_t *y) {                \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[FORM::kSmem];                        \
    FORM::template run<0>(smem, counts, xq, w, w, w, y);                                        \
  }                                                                                             \
  __global__ __launch_bounds__(FORM::kThreads) void lf_fp8_w8a8_qkv_##NAME(                    \
      const int32_t *counts, const uint8_t *xq, const uint8_t *wq, const uint8_t *wk,           \
      const uint8_t *wv, uint16_t *y) {                                                         \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[FORM::kSmem];                        \
    FORM::template run<1>(smem, counts, xq, wq, wk, wv, y);                                     \
  }                                                                                             \
  __global__ __launch_bounds__(FORM::kThreads) void lf_fp8_w8a8_gate_up_##NAME(                \
      const int32_t *counts, const uint8_t *xq, const uint8_t *wg, const uint8_t *wu,           \
      uint16_t *h) {                                                                            \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[FORM::kSmem];                        \
    FORM::template run<2>(smem, counts, xq, wg, wu, wu, h);                                     \
  }                                                                                             \
  __global__ __launch_bounds__(FORM::kThreads) void lf_fp8_w8a8_dense_##NAME##_aq(             \
      const int32_t *counts, const uint16_t *x, const uint8_t *w, uint16_t *y, uint8_t *ws) {   \
    w8a8_one_launch<FORM, 0>(counts, x, w, w, w, y, ws);                                        \
  }                                                                                             \
  __global__ __launch_bounds__(FORM::kThreads) void lf_fp8_w8a8_qkv_##NAME##_aq(               \
      const int32_t *counts, const uint16_t *x, const uint8_t *wq, const uint8_t *wk,           \
      const uint8_t *wv, uint16_t *y, uint8_t *ws) {                                            \
    w8a8_one_launch<FORM, 1>(counts, x, wq, wk, wv, y, ws);                                     \
  }                                                                                             \
  __global__ __launch_bounds__(FORM::kThreads) void lf_fp8_w8a8_gate_up_##NAME##_aq(           \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,           \
      uint16_t *h, uint8_t *ws) {                                                               \
    w8a8_one_launch<FORM, 2>(counts, x, wg, wu, wu, h, ws);                                     \
  }

LF_W8A8_ENTRIES(t256, GemmT256)
LF_W8A8_ENTRIES(t256x128, GemmT256x128)
LF_W8A8_ENTRIES(t256w8, GemmT256w8)
LF_W8A8_ENTRIES(t128, GemmT128)

// W8A8 GatedMlp in one launch: (counts, x, wg, wu, wd, y, ws), gate/up form
// then down form in the name.
#define LF_W8A8_GATED_MLP(NAME, GU, DN)                                                        \
  __global__ __launch_bounds__(GU::kThreads) void lf_fp8_w8a8_gated_mlp_##NAME(                \
      const int32_t *counts, const uint16_t *x, const uint8_t *wg, const uint8_t *wu,          \
      const uint8_t *wd, uint16_t *y, uint8_t *ws) {                                           \
    w8a8_gated_mlp<GU, DN>(counts, x, wg, wu, wd, y, ws);                                      \
  }

LF_W8A8_GATED_MLP(t256_t256, GemmT256S, GemmT256S)
LF_W8A8_GATED_MLP(t256_t256x128, GemmT256S, GemmT256x128S)
LF_W8A8_GATED_MLP(t128_t128, GemmT128S, GemmT128S)

// Block-scaled (128 x 128 weight blocks, 128-column activation groups) W8A8
// operations, one launch each: (counts, x, w..., y, ws).
__global__ __launch_bounds__(256) void lf_fp8_w8a8_dense_b128(const int32_t *counts, const uint16_t *x,
                                                              const uint8_t *w, uint16_t *y, uint8_t *ws) {
  w8a8_b128_one_launch<0>(counts, x, w, w, w, y, ws);
}
__global__ __launch_bounds__(256) void lf_fp8_w8a8_qkv_b128(const int32_t *counts, const uint16_t *x,
                                                            const uint8_t *wq, const uint8_t *wk,
                                                            const uint8_t *wv, uint16_t *y, uint8_t *ws) {
  w8a8_b128_one_launch<1>(counts, x, wq, wk, wv, y, ws);
}
__global__ __launch_bounds__(256) void lf_fp8_w8a8_gate_up_b128(const int32_t *counts, const uint16_t *x,
                                                                const uint8_t *wg, const uint8_t *wu,
                                                                uint16_t *h, uint8_t *ws) {
  w8a8_b128_one_launch<2>(counts, x, wg, wu, wu, h, ws);
}
// The same on 256 x 256 tiles (eight waves), for launches of at least 192
// such tiles (lunaflux_fp8_launch_geometry picks the form).
__global__ __launch_bounds__(512) void lf_fp8_w8a8_dense_b128_t256(const int32_t *counts, const uint16_t *x,
                                                                   const uint8_t *w, uint16_t *y, uint8_t *ws) {
  w8a8_b128_v4_one_launch<B128V4Tile, 0>(counts, x, w, w, w, y, ws);
}
__global__ __launch_bounds__(512) void lf_fp8_w8a8_qkv_b128_t256(const int32_t *counts, const uint16_t *x,
                                                                 const uint8_t *wq, const uint8_t *wk,
                                                                 const uint8_t *wv, uint16_t *y, uint8_t *ws) {
  w8a8_b128_v4_one_launch<B128V4Tile, 1>(counts, x, wq, wk, wv, y, ws);
}
__global__ __launch_bounds__(512) void lf_fp8_w8a8_gate_up_b128_t256(const int32_t *counts, const uint16_t *x,
                                                                     const uint8_t *wg, const uint8_t *wu,
                                                                     uint16_t *h, uint8_t *ws) {
  w8a8_b128_v4_one_launch<B128V4Tile, 2>(counts, x, wg, wu, wu, h, ws);
}
// The same on 256 x 128 tiles (eight waves of 32 x 128), where 256 x 256
// tiles would be too few.
__global__ __launch_bounds__(512) void lf_fp8_w8a8_dense_b128_t256x128(const int32_t *counts,
                                                                       const uint16_t *x, const uint8_t *w,
                                                                       uint16_t *y, uint8_t *ws) {
  w8a8_b128_v4_one_launch<B128V4TileN128, 0>(counts, x, w, w, w, y, ws);
}
__global__ __launch_bounds__(512) void lf_fp8_w8a8_qkv_b128_t256x128(const int32_t *counts, const uint16_t *x,
                                                                     const uint8_t *wq, const uint8_t *wk,
                                                                     const uint8_t *wv, uint16_t *y,
                                                                     uint8_t *ws) {
  w8a8_b128_v4_one_launch<B128V4TileN128, 1>(counts, x, wq, wk, wv, y, ws);
}
__global__ __launch_bounds__(512) void lf_fp8_w8a8_gate_up_b128_t256x128(const int32_t *counts,
                                                                         const uint16_t *x, const uint8_t *wg,
                                                                         const uint8_t *wu, uint16_t *h,
                                                                         uint8_t *ws) {
  w8a8_b128_v4_one_launch<B128V4TileN128, 2>(counts, x, wg, wu, wu, h, ws);
}
__global__ __launch_bounds__(256) void lf_fp8_w8a8_gated_mlp_b128(const int32_t *counts, const uint16_t *x,
                                                                  const uint8_t *wg, const uint8_t *wu,
                                                                  const uint8_t *wd, uint16_t *y,
                                                                  uint8_t *ws) {
  w8a8_b128_gated_mlp<0>(counts, x, wg, wu, wd, y, ws);
}
// The same on 256 x 256 tiles (eight waves, 256-row bands).
__global__ __launch_bounds__(512) void lf_fp8_w8a8_gated_mlp_b128_t256(const int32_t *counts,
                                                                       const uint16_t *x, const uint8_t *wg,
                                                                       const uint8_t *wu, const uint8_t *wd,
                                                                       uint16_t *y, uint8_t *ws) {
  w8a8_b128_gated_mlp<2>(counts, x, wg, wu, wd, y, ws);
}

__global__ __launch_bounds__(256) void lf_fp8_act_quant_rows(const int32_t *counts,
                                                             const uint16_t *x,
                                                             const uint8_t *w, uint8_t *xq) {
  act_quant_rows(counts, x, w, xq);
}

// RmsNorm + per-token quantizer, one entry per epsilon (the epsilon is part
// of the operation's NormalizationShape, model/plan/plan.mbt:146-151, so an
// AOT entry is built per value): 1e-5 (Llama-3) and 1e-6 (the reference
// spec's default, model/spec/llama.mbt:39).
__global__ __launch_bounds__(256) void lf_fp8_rms_norm_quant_rows_eps1em5(
    const int32_t *counts, const uint16_t *x, const uint16_t *gamma, const uint8_t *w,
    uint8_t *xq) {
  rms_norm_quant_rows(counts, x, gamma, w, xq, 1e-5f);
}
__global__ __launch_bounds__(256) void lf_fp8_rms_norm_quant_rows_eps1em6(
    const int32_t *counts, const uint16_t *x, const uint16_t *gamma, const uint8_t *w,
    uint8_t *xq) {
  rms_norm_quant_rows(counts, x, gamma, w, xq, 1e-6f);
}

}  // extern "C"
