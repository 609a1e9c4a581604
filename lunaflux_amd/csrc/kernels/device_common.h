// device_common.h - gfx950 device helpers shared by the FP8 kernels:
// vector types for the MFMA operands, the weight-region header as the device
// sees it, bf16 / e4m3 conversions, and wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

#define LF_DEVICE __device__ __forceinline__

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 in order: a loop
// whose index is a constant expression in the body, so register arrays
// indexed by it stay in registers.
template <class F, int... I>
LF_DEVICE void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
LF_DEVICE void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Mirror of lf_fp8_weight_header (include/lunaflux_fp8.h); only the fields
// the kernels read.
struct WeightHeader {
  uint32_t magic, version, layout, scale_mode;
  uint32_t rows, columns, experts, reserved;
  uint64_t tile_offset, tile_bytes, scale_offset, scale_bytes;
};

constexpr uint32_t kWeightMagic = 0x5738464Cu;
constexpr uint32_t kScalePerChannel = 1u;
constexpr uint32_t kScaleBlock128 = 2u;
// Header size = tile_offset of every region written by the host pack.
constexpr uint64_t kWeightHeaderBytes = 256;
constexpr int kTileBytes = 2048;
constexpr int kQueryTokensIndex = 3;

LF_DEVICE const WeightHeader &header_of(const uint8_t *region) {
  return *reinterpret_cast<const WeightHeader *>(region);
}

// The per-channel dense, QKV and gate/up kernels read one fp32 scale per
// output channel (s[n] for n < N); the _b128 kernels read (N/128)(K/128)
// block scales. Each refuses a region of the other scale mode (and one
// without the pack's magic) before any other read; the host admission
// rejects such a binding. MODE 1 (QKV) checks all three weights.
template <int MODE, uint32_t SCALE = kScalePerChannel>
LF_DEVICE bool dense_regions_ok(const uint8_t *w0, const uint8_t *w1, const uint8_t *w2) {
  bool ok = header_of(w0).magic == kWeightMagic && header_of(w0).scale_mode == SCALE;
  if (MODE != 0) {
    ok = ok && header_of(w1).magic == kWeightMagic && header_of(w1).scale_mode == SCALE;
  }
  if (MODE == 1) {
    ok = ok && header_of(w2).magic == kWeightMagic && header_of(w2).scale_mode == SCALE;
  }
  return ok;
}

LF_DEVICE const uint8_t *expert_tiles(const uint8_t *region, int expert) {
  const WeightHeader &h = header_of(region);
  return region + h.tile_offset + static_cast<uint64_t>(expert) * h.tile_bytes;
}

LF_DEVICE const float *expert_scales(const uint8_t *region, int expert) {
  const WeightHeader &h = header_of(region);
  return reinterpret_cast<const float *>(region + h.scale_offset +
                                         static_cast<uint64_t>(expert) * h.scale_bytes);
}

LF_DEVICE int live_rows(const int32_t *counts, int capacity) {
  int m = counts[kQueryTokensIndex];
  m = m < 0 ? 0 : m;
  return m > capacity ? capacity : m;
}

LF_DEVICE uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

// Bank swizzle of 256-byte activation rows (one bf16 k-tile of a row) in
// LDS: row r keeps 16-byte chunk c at chunk c ^ chunk_swizzle(r & 15), so
// the 16 lanes that read one logical chunk of 16 consecutive rows (an MFMA
// fragment) hit distinct banks. Measured on gfx950 with ds_read_b128 (a
// wave per pattern, 8 waves per CU): XOR with the 2-bit halves of r swapped
// reads at the contiguous rate, 256 B/clk per CU; XOR with r itself at 2/3
// of it.
LF_DEVICE int chunk_swizzle(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

LF_DEVICE float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// fp32 -> bf16 bits, round to nearest even; a NaN keeps its sign and top
// payload bits and becomes quiet: for u = the fp32 bits,
//   NaN:       (u >> 16) | 0x40
//   otherwise: (u + 0x7fff + ((u >> 16) & 1)) >> 16   (fp32 denormals kept)
// One v_cvt_pk_bf16_f32 (the conversion of a float to __bf16 on gfx950).
// It was compared with the formula above on every one of the 2^32 fp32
// inputs on MI355X under these kernels' floating-point mode, with no
// difference. The formula, compiled, is a divergent branch plus five
// integer operations per value: at 128 values per lane it cost the 256-row
// GEMM epilogues ~5 us per tile.
LF_DEVICE uint32_t f32_to_bf16(float v) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(v)));
}

// Four e4m3 codes (one 32-bit word) -> four bf16 values (two words). The
// conversion is exact: every e4m3 value is a bf16 value.
LF_DEVICE void e4m3x4_to_bf16x4(uint32_t word, uint32_t &lo, uint32_t &hi) {
  bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(word), 1.0f, false);
  bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(word), 1.0f, true);
  lo = __builtin_bit_cast(uint32_t, a);
  hi = __builtin_bit_cast(uint32_t, b);
}

// Carries the last nonzero scale forward: returns the ratio prev / s for a
// nonzero s (prev <- s), 1 otherwise.
LF_DEVICE float carry_ratio(float s, float &prev) {
  if (s == 0.0f) return 1.0f;
  const float r = prev / s;
  prev = s;
  return r;
}

// A wave-uniform read-only float through the constant address space: a
// scalar load (lgkm counter, so the vector-memory waits of a hand-counted
// load ring are not disturbed).
LF_DEVICE float sload(const float *p, int i) {
  typedef const __attribute__((address_space(4))) float cfloat;
  return ((cfloat *)p)[i];
}

LF_DEVICE float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset));
  return v;
}

// SiLU(g) * u in the reference's order, g / (1 + e^-g) * u, with the
// hardware exp2 and reciprocal (each within 1 ulp; e^-g = 2^(-g log2 e)):
// 5 instructions instead of the 28 of expf and an IEEE division, and within
// a few fp32 ulp of that form (far inside the bf16 output tolerance).
// Infinities and NaNs come out as in the IEEE form (-inf: NaN, +inf: +inf).
LF_DEVICE float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
  const float s = g * __builtin_amdgcn_rcpf(1.0f + e);
  return s * u;
}
