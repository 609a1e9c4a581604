// pack.cpp - host side of include/lunaflux_fp8.h: the weight-region format
// (header + MFMA-fragment-ordered tiles + fp32 scales), its inverse, and the
// launch geometry of every kernel entry point. No device code here.
#include "lunaflux_fp8.h"
#include "lunaflux_hip.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>

namespace {

constexpr int64_t kMaxDim = int64_t(1) << 30;

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

int64_t scale_count(int32_t mode, int64_t rows, int64_t columns) {
  return mode == LF_FP8_SCALE_PER_CHANNEL ? rows : (rows / 128) * (columns / 128);
}

bool shape_ok(int32_t mode, int64_t rows, int64_t columns, int32_t experts) {
  if (rows <= 0 || columns <= 0 || experts <= 0 || rows > kMaxDim ||
      columns > kMaxDim || experts > 4096) {
    return false;
  }
  if (rows % LF_FP8_TILE_ROWS != 0 || columns % LF_FP8_TILE_COLUMNS != 0) return false;
  if (mode == LF_FP8_SCALE_BLOCK128) return rows % 128 == 0;
  return mode == LF_FP8_SCALE_PER_CHANNEL;
}

void fill_header(lf_fp8_weight_header *h, int32_t mode, int64_t rows,
                 int64_t columns, int32_t experts) {
  std::memset(h, 0, sizeof(*h));
  h->magic = LF_FP8_WEIGHT_MAGIC;
  h->version = LF_FP8_WEIGHT_VERSION;
  h->layout = LF_FP8_LAYOUT_TILE16X128;
  h->scale_mode = static_cast<uint32_t>(mode);
  h->rows = static_cast<uint32_t>(rows);
  h->columns = static_cast<uint32_t>(columns);
  h->experts = static_cast<uint32_t>(experts);
  h->tile_offset = LF_FP8_HEADER_BYTES;
  h->tile_bytes = static_cast<uint64_t>(rows * columns);
  h->scale_offset = h->tile_offset + h->tile_bytes * static_cast<uint64_t>(experts);
  h->scale_bytes = static_cast<uint64_t>(align_up(scale_count(mode, rows, columns) * 4, 256));
}

// Byte offset, inside one expert's tile block, of W[n][k].
inline int64_t swizzled_offset(int64_t n, int64_t k, int64_t columns) {
  int64_t nt = n / 16, r = n % 16;
  int64_t kt = k / 128, kk = k % 128;
  int64_t g = kk / 32, h = (kk % 32) / 16, b = kk % 16;
  int64_t lane = g * 16 + r;
  return (nt * (columns / 128) + kt) * LF_FP8_TILE_BYTES + h * 1024 + lane * 16 + b;
}


// W8A16 work split (the kernels are in lunaflux_amd/csrc/kernels/w8a16.hip).
// Profiles with at most 16 rows use the one-tile form: a block of
// kW16TileWaves waves per 16-column tile, K split across its waves, one
// block per tile. Larger profiles use the column-group form: one tile per
// wave, kW16Waves tiles per block, K cut into `split` slices across blocks
// (about 512 blocks: two per CU of an MI355X, which is what its 64 KiB LDS
// ring allows), partial tiles reduced through the workspace. Measured at
// M = 32 on the Llama-3-8B shapes: 256 or 768+ blocks are slower (fewer
// bytes in flight, or more partial traffic).
constexpr int kW16Waves = 4;
constexpr int kW16TileWaves = 8;
struct W8a16Split {
  int mt;
  bool one_tile;
  int64_t groups, split;
};
bool w8a16_split(int64_t n, int64_t k, int32_t max_tokens, W8a16Split *out) {
  if (n % 16 != 0 || max_tokens > 128) return false;
  const int mt = max_tokens <= 16 ? 1 : max_tokens <= 32 ? 2 : max_tokens <= 64 ? 4 : 8;
  const int64_t kt = k / 128, tiles = n / 16;
  out->mt = mt;
  out->one_tile = mt == 1;
  if (out->one_tile) {
    out->groups = tiles;
    out->split = 1;
    return tiles <= INT32_MAX;
  }
  const int64_t groups = (tiles + kW16Waves - 1) / kW16Waves;
  int64_t split = (512 + groups / 2) / groups;
  if (split < 1) split = 1;
  if (split > kt) split = kt;
  if (groups * split > INT32_MAX) return false;
  out->groups = groups;
  out->split = split;
  return true;
}

// Block-scaled W8A16 entries (_B128): profiles of 65..128 rows take the
// LDS-tiled GEMM form with the per-channel entries' tile and split
// (w8a16_gemm below, the _b128_m128_n{BN} symbols; every block-scaled width
// is a multiple of 128, so a 16-column fragment lies in one 128-row scale
// block); every other profile (also <= 16 rows) the column-group form,
// split as above, with at least enough slices that each holds <= 128
// k-tiles (the block scales of a slice are staged in LDS, kW16BlockSliceKT
// in kernels/w8a16.hip).
bool w8a16_b128_entry(int32_t e) {
  return e == LF_FP8_ENTRY_W8A16_DENSE_B128 || e == LF_FP8_ENTRY_W8A16_QKV_B128 ||
         e == LF_FP8_ENTRY_W8A16_GATE_UP_B128;
}
// The per-channel entry whose tile and split rules a block-scaled one shares.
int32_t w8a16_channel_entry(int32_t e) {
  return e == LF_FP8_ENTRY_W8A16_DENSE_B128 ? LF_FP8_ENTRY_W8A16_DENSE
         : e == LF_FP8_ENTRY_W8A16_QKV_B128 ? LF_FP8_ENTRY_W8A16_QKV
                                             : LF_FP8_ENTRY_W8A16_GATE_UP;
}
bool w8a16_b128_split(int64_t n, int64_t k, int32_t max_tokens, W8a16Split *out) {
  if (n % 128 != 0 || k % 128 != 0 || !w8a16_split(n, k, max_tokens, out)) return false;
  const int64_t kt = k / 128, tiles = n / 16;
  if (out->one_tile) {
    out->one_tile = false;
    out->groups = (tiles + kW16Waves - 1) / kW16Waves;
    out->split = std::min<int64_t>(kt, std::max<int64_t>(1, (512 + out->groups / 2) / out->groups));
  }
  out->split = std::max<int64_t>(out->split, (kt + 127) / 128);
  return out->groups * out->split <= INT32_MAX;
}

// Shape-specialized W8A16 entries (w8a16.hip, "LF_W16_FIXED_*"): compiled for
// one input width K (and, for QKV, one Q / K-V split), as AOT entry points
// are compiled for one model shape. Two forms: one-tile (a block of `waves`
// waves per 16-column tile, K split across its waves, no workspace) and
// column-group (`waves` tiles per block, K cut into `split` slices across
// blocks, partials reduced through the workspace). Shapes without an entry
// here use the generic kernels above.
struct W8a16Fixed {
  int32_t entry;
  int64_t k, nq, nkv;
  int mt;           // 16-row tiles: the profile's max_query_tokens <= 16 mt
  bool group;       // column-group form
  int waves, split;
  const char *symbol;
  int64_t min_n = 0;  // chosen only for N >= min_n (earlier rows win)
};
constexpr int64_t kWideN = 16384;
constexpr W8a16Fixed kW8a16Fixed[] = {
    {LF_FP8_ENTRY_W8A16_DENSE, 4096, 0, 0, 1, true, 2, 1, "lf_fp8_w8a16_dense_wide_k4096_m16", kWideN},
    {LF_FP8_ENTRY_W8A16_DENSE, 4096, 0, 0, 2, true, 4, 1, "lf_fp8_w8a16_dense_wide_k4096_m32", kWideN},
    {LF_FP8_ENTRY_W8A16_DENSE, 4096, 0, 0, 8, true, 8, 1, "lf_fp8_w8a16_dense_wide_k4096_m128", kWideN},
    {LF_FP8_ENTRY_W8A16_DENSE, 4096, 0, 0, 1, false, 8, 1, "lf_fp8_w8a16_dense_k4096_m16"},
    {LF_FP8_ENTRY_W8A16_DENSE, 4096, 0, 0, 2, false, 8, 1, "lf_fp8_w8a16_dense_k4096_m32"},
    {LF_FP8_ENTRY_W8A16_DENSE, 14336, 0, 0, 1, false, 8, 1, "lf_fp8_w8a16_dense_k14336_m16"},
    {LF_FP8_ENTRY_W8A16_DENSE, 14336, 0, 0, 2, true, 4, 4, "lf_fp8_w8a16_dense_k14336_m32"},
    {LF_FP8_ENTRY_W8A16_QKV, 4096, 4096, 1024, 1, false, 8, 1,
     "lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m16"},
    {LF_FP8_ENTRY_W8A16_QKV, 4096, 4096, 1024, 2, true, 8, 4,
     "lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m32"},
    {LF_FP8_ENTRY_W8A16_GATE_UP, 4096, 0, 0, 1, true, 2, 1, "lf_fp8_w8a16_gate_up_k4096_m16"},
    {LF_FP8_ENTRY_W8A16_GATE_UP, 4096, 0, 0, 2, true, 4, 1, "lf_fp8_w8a16_gate_up_k4096_m32"},
    // the same forms over 128 x 128 block-scaled weights (no wide entries)
    {LF_FP8_ENTRY_W8A16_DENSE_B128, 4096, 0, 0, 1, false, 8, 1, "lf_fp8_w8a16_dense_b128_k4096_m16"},
    {LF_FP8_ENTRY_W8A16_DENSE_B128, 4096, 0, 0, 2, false, 8, 1, "lf_fp8_w8a16_dense_b128_k4096_m32"},
    {LF_FP8_ENTRY_W8A16_DENSE_B128, 14336, 0, 0, 1, false, 8, 1, "lf_fp8_w8a16_dense_b128_k14336_m16"},
    {LF_FP8_ENTRY_W8A16_DENSE_B128, 14336, 0, 0, 2, true, 4, 4, "lf_fp8_w8a16_dense_b128_k14336_m32"},
    {LF_FP8_ENTRY_W8A16_QKV_B128, 4096, 4096, 1024, 1, false, 8, 1,
     "lf_fp8_w8a16_qkv_b128_k4096_q4096_kv1024_m16"},
    {LF_FP8_ENTRY_W8A16_QKV_B128, 4096, 4096, 1024, 2, true, 8, 4,
     "lf_fp8_w8a16_qkv_b128_k4096_q4096_kv1024_m32"},
    {LF_FP8_ENTRY_W8A16_GATE_UP_B128, 4096, 0, 0, 1, true, 2, 1, "lf_fp8_w8a16_gate_up_b128_k4096_m16"},
    {LF_FP8_ENTRY_W8A16_GATE_UP_B128, 4096, 0, 0, 2, true, 4, 1, "lf_fp8_w8a16_gate_up_b128_k4096_m32"},
};

// The specialized entry for (entry, N, K, Q / K-V split, profile), or null.
// nq = nkv = 0 when the split is unknown (QKV then never matches).
const W8a16Fixed *w8a16_fixed(int32_t entry, int64_t n, int64_t k, int64_t nq, int64_t nkv,
                              int32_t max_tokens) {
  if (max_tokens <= 0 || max_tokens > 128 || n <= 0 || n % 16 != 0) return nullptr;
  // the profile's 16-row fragments (profiles of 33..64 rows have no entries)
  const int mt = max_tokens <= 16 ? 1 : max_tokens <= 32 ? 2 : max_tokens <= 64 ? 4 : 8;
  for (const W8a16Fixed &f : kW8a16Fixed) {
    if (f.entry != entry || f.k != k || f.mt != mt || n < f.min_n) continue;
    if ((entry == LF_FP8_ENTRY_W8A16_QKV || entry == LF_FP8_ENTRY_W8A16_QKV_B128) &&
        (f.nq != nq || f.nkv != nkv || n != nq + 2 * nkv)) {
      continue;
    }
    if (f.group && (n / 16) % f.waves != 0) continue;
    return &f;
  }
  return nullptr;
}

int64_t w8a16_fixed_workspace(const W8a16Fixed &f, int64_t n) {
  if (!f.group || f.split == 1) return 256;
  const int64_t nw = f.entry == LF_FP8_ENTRY_W8A16_GATE_UP || f.entry == LF_FP8_ENTRY_W8A16_GATE_UP_B128 ? 2 : 1;
  const int64_t groups = n / 16 / f.waves;
  return align_up(f.split * (n / 16) * nw * f.mt * 1024, 256) + align_up(groups * 4, 256);
}

void w8a16_fixed_geometry(const W8a16Fixed &f, int64_t n, int32_t *gx, int32_t *bx) {
  const int64_t tiles = n / 16;
  *gx = static_cast<int32_t>(f.group ? tiles / f.waves * f.split : tiles);
  *bx = 64 * f.waves;
}

// Profiles of 65..128 rows: the LDS-tiled GEMM (kernels/w8a16_gemm.hip,
// "lf_fp8_w8a16_{op}_m128_n{BN}"), any K, any N its blocks divide. A block
// (8 waves) computes 128 rows x BN weight columns (gate/up: BN / 2 gate and
// BN / 2 up columns) over one of S K-slices. Among BN 64 and 128 and the
// splits that keep >= 8 k-tiles per slice, the most blocks up to one per CU
// (256), the smaller split on a tie (at equal blocks BN 64 has half the
// slices, so half the partials; over 128 x 128 block-scaled weights BN 128
// on a tie, see below); with no such choice (more than 256 column
// blocks even unsplit) BN 128 unsplit. Measured at M = 128 on the
// Llama-3-8B shapes (MI355X, 24 weight copies rotated so the MALL serves
// none), each call under several geometries on one box: QKV (64, 2)
// 18.4-19.2 us against (128, 4) 19.9-21.5, down (64, 4) 28.9-31.0 against
// (128, 6) 31.3-34.2 and (64, 3) 33.6-36.6, o (64, 4) 14.3-14.9 against
// (64, 3) 14.4-15.2, gate/up (128, 1) 38.6-40.2 against (64, 1) 55.7-59.5
// (448 blocks). Block-scaled weights (block = true; the per-k-step scale
// fold) measured the other way at equal blocks, layer loop A/B: QKV
// (128, 4) 21.1-21.3 us against (64, 2) 23.3-24.0, down (128, 6) 34.8-36.2
// against (64, 4) 39.3-40.2, o (64, 4) 16.0-16.4 against (64, 3) 17.9-19.1.
// Vocabulary-wide dense shapes with a column-group entry keep it.
struct W8a16Gemm {
  int bn;
  int64_t blocks_n, split;
};
bool w8a16_gemm(int32_t entry, int64_t n, int64_t k, int32_t max_tokens, W8a16Gemm *out,
                bool block = false) {
  if (max_tokens <= 64 || max_tokens > 128 || n <= 0 || k <= 0 || k % 128 != 0) return false;
  if (entry == LF_FP8_ENTRY_W8A16_DENSE && n >= kWideN &&
      w8a16_fixed(entry, n, k, 0, 0, max_tokens) != nullptr) {
    return false;
  }
  const int64_t kt = k / 128;
  constexpr int64_t kMaxBlocks = 256, kMinSliceTiles = 8;
  const int64_t max_split = std::max<int64_t>(1, kt / kMinSliceTiles);
  W8a16Gemm best{0, 0, 0};
  const int order[2] = {block ? 128 : 64, block ? 64 : 128};
  for (const int bn : order) {
    const int64_t per = entry == LF_FP8_ENTRY_W8A16_GATE_UP ? bn / 2 : bn;
    if (n % per != 0) continue;
    const int64_t blocks = n / per;
    const int64_t split = std::min(max_split, std::max<int64_t>(1, kMaxBlocks / blocks));
    if (blocks * split > kMaxBlocks) continue;
    // the first width keeps a tie
    if (blocks * split > best.blocks_n * best.split) best = W8a16Gemm{bn, blocks, split};
  }
  if (best.bn == 0) {
    for (const int bn : {128, 64}) {
      const int64_t per = entry == LF_FP8_ENTRY_W8A16_GATE_UP ? bn / 2 : bn;
      if (n % per == 0) {
        best = W8a16Gemm{bn, n / per, 1};
        break;
      }
    }
    if (best.bn == 0) return false;
  }
  *out = best;
  return best.blocks_n * best.split <= INT32_MAX;
}

// One-launch GatedMlp entries (kernels/w8a16.hip, LF_W16_GATED_MLP): the
// profile's gate/up and down column-group parameters. Workspace: h [16 mt
// rows][I] bf16, the down kernel's split-K partials and arrival counters,
// then 768 bytes: the slice counters and the done counter and error word,
// one 128-byte line each (the error word in the last line but one).
struct W8a16Gated {
  int64_t hidden, inter;
  int mt, waves, down_split;
  const char *symbol;
  bool block = false;  // 128 x 128 block-scaled weights (LF_FP8_ENTRY_W8A16_GATED_MLP_B128)
};
constexpr W8a16Gated kW8a16Gated[] = {
    {4096, 14336, 1, 4, 4, "lf_fp8_w8a16_gated_mlp_h4096_i14336_m16"},
    {4096, 14336, 2, 4, 4, "lf_fp8_w8a16_gated_mlp_h4096_i14336_m32"},
    {4096, 14336, 1, 4, 4, "lf_fp8_w8a16_gated_mlp_b128_h4096_i14336_m16", true},
    {4096, 14336, 2, 4, 4, "lf_fp8_w8a16_gated_mlp_b128_h4096_i14336_m32", true},
};

bool w8a16_gated_entry(int32_t entry) {
  return entry == LF_FP8_ENTRY_W8A16_GATED_MLP || entry == LF_FP8_ENTRY_W8A16_GATED_MLP_B128;
}

const W8a16Gated *w8a16_gated(int32_t entry, int64_t hidden, int64_t inter, int32_t max_tokens) {
  if (!w8a16_gated_entry(entry) || max_tokens <= 0 || max_tokens > 32) return nullptr;
  const int mt = max_tokens <= 16 ? 1 : 2;
  const bool block = entry == LF_FP8_ENTRY_W8A16_GATED_MLP_B128;
  for (const W8a16Gated &g : kW8a16Gated) {
    if (g.hidden == hidden && g.inter == inter && g.mt == mt && g.block == block) return &g;
  }
  return nullptr;
}

int64_t w8a16_gated_workspace(const W8a16Gated &g) {
  const int64_t h = align_up(16 * g.mt * g.inter * 2, 256);
  const int64_t tiles = g.hidden / 16;
  const int64_t down = align_up(g.down_split * tiles * g.mt * 1024, 256) +
                       align_up(tiles / g.waves * 4, 256);
  return h + down + 768;
}

// W8A8 tile forms (kernels/projection.hip). Output columns per block: BN
// for dense / QKV, BN / 2 h-columns for gate/up (a block computes BN / 2
// gate and BN / 2 up columns). 256 x 256 tiles when the launch has at least
// 192 of them (three quarters of a tile per CU of the 256 on an MI355X) and
// the columns divide: on 4 waves (t256) from 256 tiles, on 8 waves (t256w8,
// a single tile per CU, whose load latency two waves per SIMD hide better)
// below that. Fewer: QKV and dense on 256 x 128 tiles (4 waves, t256x128)
// when those number 128-256 (at most one per CU); otherwise 128 x 128 tiles
// (4 waves, two blocks per CU). Measured at M = 2048: QKV (192 large tiles)
// 71.2 -> 59.5 us on the large tiles; o and down (128) were 30-40 % slower
// on them and 9-10 % faster on 256 x 128 than on 128 x 128.
// The 256-row forms address a tile's activation rows with 32-bit offsets
// from its first row, which needs 256 K < 2^32; wider K takes 128 x 128.
enum class W8a8Form { kT256, kT256w8, kT256x128, kT128 };
struct W8a8Tiles {
  W8a8Form form;
  int bm, bn, threads;
  int64_t gx, bands;  // column blocks, row bands (of bm rows) for the profile
};
const char *w8a8_form_name(W8a8Form f) {
  switch (f) {
    case W8a8Form::kT256: return "t256";
    case W8a8Form::kT256w8: return "t256w8";
    case W8a8Form::kT256x128: return "t256x128";
    default: return "t128";
  }
}
W8a8Tiles w8a8_tiles_of(W8a8Form f, bool gate_up, int64_t n, int32_t max_tokens) {
  W8a8Tiles t{f, 256, 256, 256, 0, 0};
  if (f == W8a8Form::kT256w8) t.threads = 512;
  if (f == W8a8Form::kT256x128) t.bn = 128;
  if (f == W8a8Form::kT128) t.bm = t.bn = 128;
  t.gx = n / (gate_up ? t.bn / 2 : t.bn);
  t.bands = (max_tokens + t.bm - 1) / t.bm;
  return t;
}
// false if no form takes the shape (n not a multiple of the 128-column form's
// block width).
bool w8a8_tiles(bool gate_up, int64_t n, int64_t k, int32_t max_tokens, W8a8Tiles *out) {
  const int64_t cols256 = gate_up ? 128 : 256, cols128 = gate_up ? 64 : 128;
  if (n % cols128 != 0) return false;
  const bool offsets32 = k < (int64_t(1) << 24);
  const int64_t bands256 = (max_tokens + 255) / 256;
  const int64_t tiles256 = (n % cols256 == 0 && offsets32) ? bands256 * (n / cols256) : 0;
  const int64_t tiles256x128 = !gate_up && offsets32 ? bands256 * (n / cols128) : 0;
  const bool big = tiles256 >= 192, four_wave = tiles256 >= 256;
  const bool wide128 = !big && tiles256x128 >= 128 && tiles256x128 <= 256;
  const W8a8Form f = big ? (four_wave ? W8a8Form::kT256 : W8a8Form::kT256w8)
                         : wide128 ? W8a8Form::kT256x128 : W8a8Form::kT128;
  *out = w8a8_tiles_of(f, gate_up, n, max_tokens);
  return true;
}

// One-launch W8A8 entries (_aq, and the GatedMlp): 256 quantizer blocks
// per quantizer step ahead of the GEMM blocks (kQuantBlocks in
// kernels/projection.hip), and the sync area of kernels/phases.h at the
// start of the workspace.
constexpr int64_t kQuantBlocks = 256;
// (kernels/phases.h: error word, done counter, then one 128-byte line per
// band counter)
int64_t sync_bytes(int64_t steps, int64_t bands) { return 256 + 128 * steps * bands; }
int64_t quantized_rows_bytes(int64_t rows, int64_t k) {
  return align_up(rows * k, 256) + align_up(rows * 4, 256);
}

// Block-scaled W8A8 entries (kernels/projection.hip, _b128): 128 x 128 tiles
// of 4 waves after kQuantBlocks group-quantizer blocks; the quantized rows
// hold codes [cap, K] then the group scales k-tile-major [K / 128][cap].
bool w8a8_b128_entry(int32_t e) {
  return e == LF_FP8_ENTRY_W8A8_DENSE_B128 || e == LF_FP8_ENTRY_W8A8_QKV_B128 ||
         e == LF_FP8_ENTRY_W8A8_GATE_UP_B128;
}
int64_t b128_rows_bytes(int64_t cap, int64_t k) {
  return align_up(cap * k, 256) + align_up((k / 128) * cap * 4, 256);
}
// Row bands of 128 for the profile; false if the shape has no form (widths
// not multiples of 128, or group-scale indices past int32).
bool w8a8_b128_bands(int64_t n, int64_t k, int32_t max_tokens, int64_t *bands) {
  if (n <= 0 || k <= 0 || n % 128 != 0 || k % 128 != 0 || max_tokens <= 0) return false;
  *bands = (max_tokens + 127) / 128;
  return (k / 128) * (*bands * 128) < INT32_MAX;
}
// The standalone block-scaled entries run 256-row bands on 8 waves: 256 x
// 256 tiles (_b128_t256) for profiles of at least kB128T256Tiles such tiles
// where the width is a multiple of that tile (256 columns; gate/up: 128
// outputs), else 256 x 128 tiles (_b128_t256x128; faster than 128 x 128 at
// every profile measured, 128-8192 rows). Both use 32-bit activation
// offsets (K < 2^24); past that, 128 x 128 tiles of 4 waves (_b128).
constexpr int64_t kB128T256Tiles = 192;
struct W8a8B128 {
  int form;               // 0: 128 x 128, 1: 256 x 128, 2: 256 x 256
  int64_t bm, gx, bands;  // band height, column blocks, row bands
};
const char *w8a8_b128_suffix(int form) { return form == 2 ? "_t256" : form == 1 ? "_t256x128" : ""; }
bool w8a8_b128_tiles(bool gate_up, int64_t n, int64_t k, int32_t max_tokens, W8a8B128 *out) {
  if (n <= 0 || k <= 0 || n % 128 != 0 || k % 128 != 0 || max_tokens <= 0) return false;
  const int64_t cols256 = gate_up ? 128 : 256;
  const bool offsets32 = k < (int64_t(1) << 24);
  const int64_t tiles256 = n % cols256 == 0 && offsets32 ? (max_tokens + 255) / 256 * (n / cols256) : 0;
  out->form = tiles256 >= kB128T256Tiles ? 2 : offsets32 ? 1 : 0;
  out->bm = out->form != 0 ? 256 : 128;
  out->gx = out->form == 2 ? n / cols256 : n / (cols256 / 2);
  out->bands = (max_tokens + out->bm - 1) / out->bm;
  return (k / 128) * (out->bands * out->bm) < INT32_MAX;
}

// Block-scaled W8A8 GatedMlp in one launch: both GEMMs on one tile form and
// band height, 256 x 256 (_t256, 512 threads) where the gate/up launch of
// the shape takes it and the hidden width is a multiple of 256, else 128 x
// 128 (no 256 x 128 form here: kernels/projection.hip, B128Form). (Llama-3-
// 8B widths, one launch: 256 x 256 270.6 / 548.1 us against 288.9 / 659.3
// on 128 x 128 at 512 / 2048 rows; 128 x 128 ahead at 128 rows.)
// out: the form, band height, the gate/up plus down column blocks and the
// bands.
bool w8a8_b128_gated(int64_t hidden, int64_t inter, int32_t max_tokens, W8a8B128 *out) {
  int64_t bands = 0;
  W8a8B128 up;
  if (!w8a8_b128_bands(hidden, inter, max_tokens, &bands) || !w8a8_b128_bands(inter, hidden, max_tokens, &bands) ||
      !w8a8_b128_tiles(true, inter, hidden, max_tokens, &up)) {
    return false;
  }
  const bool offsets32 = hidden < (int64_t(1) << 24) && inter < (int64_t(1) << 24);
  out->form = up.form == 2 && hidden % 256 == 0 && offsets32 ? 2 : 0;
  out->bm = out->form != 0 ? 256 : 128;
  const int64_t bn = out->form == 2 ? 256 : 128;
  out->gx = inter / (bn / 2) + hidden / bn;
  out->bands = (max_tokens + out->bm - 1) / out->bm;
  const int64_t cap = out->bands * out->bm;
  return (hidden / 128) * cap < INT32_MAX && (inter / 128) * cap < INT32_MAX;
}

// W8A8 GatedMlp in one launch: both GEMMs on 4-wave blocks of one band
// height. Gate/up on 256 x 256 tiles where its own launch would take 256-row
// tiles (down then on 256 x 256, or 256 x 128 where its own launch would
// not take 256 x 256), else both on 128 x 128.
struct W8a8Gated {
  W8a8Tiles gu, dn;
};
bool w8a8_gated(int64_t hidden, int64_t inter, int32_t max_tokens, W8a8Gated *out) {
  W8a8Tiles gu, dn;
  if (!w8a8_tiles(true, inter, hidden, max_tokens, &gu) || !w8a8_tiles(false, hidden, inter, max_tokens, &dn)) {
    return false;
  }
  const bool offsets32 = hidden < (int64_t(1) << 24) && inter < (int64_t(1) << 24);
  if (gu.form != W8a8Form::kT128 && offsets32 && hidden % 128 == 0) {
    out->gu = w8a8_tiles_of(W8a8Form::kT256, true, inter, max_tokens);
    const bool dn256 = (dn.form == W8a8Form::kT256 || dn.form == W8a8Form::kT256w8) && hidden % 256 == 0;
    out->dn = w8a8_tiles_of(dn256 ? W8a8Form::kT256 : W8a8Form::kT256x128, false, hidden, max_tokens);
  } else {
    out->gu = w8a8_tiles_of(W8a8Form::kT128, true, inter, max_tokens);
    out->dn = w8a8_tiles_of(W8a8Form::kT128, false, hidden, max_tokens);
  }
  return true;
}
int64_t w8a8_gated_workspace(const W8a8Gated &g, int64_t hidden, int64_t inter) {
  const int64_t cap = g.gu.bands * g.gu.bm;
  return sync_bytes(3, g.gu.bands) + quantized_rows_bytes(cap, hidden) + align_up(cap * inter * 2, 256) +
         quantized_rows_bytes(cap, inter);
}

int64_t w8a16_gemm_workspace(const W8a16Gemm &g);

// One-launch W8A16 GatedMlp for profiles of 65..128 rows (kernels/
// w8a16_gemm.hip, GatedMlpGemm): where the gate/up launch would take the
// n128 tiles unsplit, the gate/up blocks and the down launch's blocks (its
// own tile and split) in one grid. Workspace: h [128][I] bf16, the down
// GEMM's workspace, 256 bytes of count, done counter and error word.
struct W8a16GatedGemm {
  W8a16Gemm gu, dn;
};
bool w8a16_gated_gemm(int32_t entry, int64_t hidden, int64_t inter, int32_t max_tokens,
                      W8a16GatedGemm *out) {
  if (!w8a16_gated_entry(entry) || max_tokens <= 64 || max_tokens > 128) return false;
  const bool block = entry == LF_FP8_ENTRY_W8A16_GATED_MLP_B128;
  if (!w8a16_gemm(LF_FP8_ENTRY_W8A16_GATE_UP, inter, hidden, max_tokens, &out->gu, block) ||
      !w8a16_gemm(LF_FP8_ENTRY_W8A16_DENSE, hidden, inter, max_tokens, &out->dn, block)) {
    return false;
  }
  return out->gu.bn == 128 && out->gu.split == 1;
}
int64_t w8a16_gated_gemm_workspace(const W8a16GatedGemm &g, int64_t inter) {
  // sync: one 128-byte line per down K-slice counter, done, error, one spare
  return align_up(128 * inter * 2, 256) + w8a16_gemm_workspace(g.dn) + 128 * g.dn.split + 256;
}

int64_t w8a16_gemm_workspace(const W8a16Gemm &g) {
  if (g.split == 1) return 256;
  // one 1 KiB fp32 fragment per (slice, column block, wave, fragment): 8
  // waves of 2 x BN / 32 fragments; then one arrival counter per block
  const int64_t frags = 2 * (g.bn / 32);
  return align_up(g.split * g.blocks_n * 8 * frags * 1024, 256) + align_up(g.blocks_n * 4, 256);
}
}  // namespace

static_assert(sizeof(lf_fp8_weight_header) == LF_FP8_HEADER_BYTES, "header size");

extern "C" {

int32_t lunaflux_fp8_weight_region_bytes(int32_t scale_mode, int64_t rows,
                                         int64_t columns, int32_t experts,
                                         int64_t *byte_count) {
  if (byte_count == nullptr || !shape_ok(scale_mode, rows, columns, experts)) {
    return LF_INVALID_ARGUMENT;
  }
  lf_fp8_weight_header h;
  fill_header(&h, scale_mode, rows, columns, experts);
  *byte_count = static_cast<int64_t>(h.scale_offset + h.scale_bytes * static_cast<uint64_t>(experts));
  return LF_OK;
}

int32_t lunaflux_fp8_pack_weight(int32_t scale_mode, int64_t rows,
                                 int64_t columns, int32_t experts,
                                 const uint8_t *q, int64_t q_bytes,
                                 const float *scales, int64_t scale_count_arg,
                                 uint8_t *region, int64_t region_bytes) {
  int64_t need = 0;
  int32_t st = lunaflux_fp8_weight_region_bytes(scale_mode, rows, columns, experts, &need);
  if (st != LF_OK) return st;
  int64_t sc = scale_count(scale_mode, rows, columns);
  // Both source spans are checked against the shape before anything is read.
  if (q == nullptr || scales == nullptr || region == nullptr || region_bytes != need ||
      q_bytes != experts * rows * columns || scale_count_arg != experts * sc) {
    return LF_INVALID_ARGUMENT;
  }
  lf_fp8_weight_header h;
  fill_header(&h, scale_mode, rows, columns, experts);
  std::memset(region, 0, static_cast<size_t>(region_bytes));
  std::memcpy(region, &h, sizeof(h));
  for (int32_t e = 0; e < experts; e += 1) {
    const uint8_t *qe = q + e * rows * columns;
    uint8_t *te = region + h.tile_offset + static_cast<uint64_t>(e) * h.tile_bytes;
    for (int64_t n = 0; n < rows; n += 1) {
      for (int64_t k0 = 0; k0 < columns; k0 += 16) {
        // 16 consecutive k stay contiguous in the swizzled order.
        std::memcpy(te + swizzled_offset(n, k0, columns), qe + n * columns + k0, 16);
      }
    }
    std::memcpy(region + h.scale_offset + static_cast<uint64_t>(e) * h.scale_bytes,
                scales + e * sc, static_cast<size_t>(sc) * sizeof(float));
  }
  return LF_OK;
}

int32_t lunaflux_fp8_unpack_weight(const uint8_t *region, int64_t region_bytes,
                                   uint8_t *q, int64_t q_bytes, float *scales,
                                   int64_t scale_count_arg) {
  if (region == nullptr || region_bytes < LF_FP8_HEADER_BYTES) return LF_INVALID_ARGUMENT;
  lf_fp8_weight_header h;
  std::memcpy(&h, region, sizeof(h));
  if (h.magic != LF_FP8_WEIGHT_MAGIC || h.version != LF_FP8_WEIGHT_VERSION ||
      h.layout != LF_FP8_LAYOUT_TILE16X128) {
    return LF_INVALID_ARGUMENT;
  }
  int32_t mode = static_cast<int32_t>(h.scale_mode);
  int64_t rows = h.rows, columns = h.columns;
  int32_t experts = static_cast<int32_t>(h.experts);
  int64_t need = 0;
  if (lunaflux_fp8_weight_region_bytes(mode, rows, columns, experts, &need) != LF_OK ||
      need != region_bytes) {
    return LF_INVALID_ARGUMENT;
  }
  int64_t sc = scale_count(mode, rows, columns);
  if (q == nullptr || scales == nullptr || q_bytes != experts * rows * columns ||
      scale_count_arg != experts * sc) {
    return LF_INVALID_ARGUMENT;
  }
  for (int32_t e = 0; e < experts; e += 1) {
    uint8_t *qe = q + e * rows * columns;
    const uint8_t *te = region + h.tile_offset + static_cast<uint64_t>(e) * h.tile_bytes;
    for (int64_t n = 0; n < rows; n += 1) {
      for (int64_t k0 = 0; k0 < columns; k0 += 16) {
        std::memcpy(qe + n * columns + k0, te + swizzled_offset(n, k0, columns), 16);
      }
    }
    std::memcpy(scales + e * sc,
                region + h.scale_offset + static_cast<uint64_t>(e) * h.scale_bytes,
                static_cast<size_t>(sc) * sizeof(float));
  }
  return LF_OK;
}

int32_t lunaflux_fp8_admit_weight(int32_t entry, const uint8_t *region_head, int64_t head_bytes,
                                  int64_t region_bytes, int64_t rows, int64_t columns,
                                  int32_t experts) {
  const bool dense = entry == LF_FP8_ENTRY_W8A16_DENSE || entry == LF_FP8_ENTRY_W8A16_QKV ||
                     entry == LF_FP8_ENTRY_W8A16_GATE_UP || entry == LF_FP8_ENTRY_W8A8_DENSE ||
                     entry == LF_FP8_ENTRY_W8A8_QKV || entry == LF_FP8_ENTRY_W8A8_GATE_UP ||
                     entry == LF_FP8_ENTRY_W8A16_GATED_MLP || entry == LF_FP8_ENTRY_W8A8_DENSE_AQ ||
                     entry == LF_FP8_ENTRY_W8A8_QKV_AQ || entry == LF_FP8_ENTRY_W8A8_GATE_UP_AQ ||
                     entry == LF_FP8_ENTRY_W8A8_GATED_MLP;
  const bool block = w8a16_b128_entry(entry) || w8a8_b128_entry(entry) ||
                     entry == LF_FP8_ENTRY_W8A8_GATED_MLP_B128 || entry == LF_FP8_ENTRY_W8A16_GATED_MLP_B128;
  const bool grouped = entry == LF_FP8_ENTRY_GROUPED;
  if ((!dense && !block && !grouped) || region_head == nullptr || head_bytes < LF_FP8_HEADER_BYTES ||
      ((dense || block) && experts != 1)) {
    return LF_INVALID_ARGUMENT;
  }
  lf_fp8_weight_header h;
  std::memcpy(&h, region_head, sizeof(h));
  if (h.magic != LF_FP8_WEIGHT_MAGIC || h.version != LF_FP8_WEIGHT_VERSION ||
      h.layout != LF_FP8_LAYOUT_TILE16X128 || h.rows != rows || h.columns != columns ||
      h.experts != static_cast<uint32_t>(experts)) {
    return LF_INVALID_ARGUMENT;
  }
  const int32_t mode = static_cast<int32_t>(h.scale_mode);
  int64_t need = 0;
  if (lunaflux_fp8_weight_region_bytes(mode, rows, columns, experts, &need) != LF_OK) {
    return LF_INVALID_ARGUMENT;
  }
  // Every offset and size in the header must be the format's own, and the
  // region exactly the format's size: the specialized entries issue their
  // weight loads before they read the header, so this check is what keeps
  // them inside the region.
  lf_fp8_weight_header want;
  fill_header(&want, mode, rows, columns, experts);
  if (region_bytes != need || h.tile_offset != want.tile_offset ||
      h.tile_bytes != want.tile_bytes || h.scale_offset != want.scale_offset ||
      h.scale_bytes != want.scale_bytes) {
    return LF_INVALID_ARGUMENT;
  }
  if (dense && mode != LF_FP8_SCALE_PER_CHANNEL) return LF_UNSUPPORTED;
  if (block && mode != LF_FP8_SCALE_BLOCK128) return LF_UNSUPPORTED;
  return LF_OK;
}

int64_t lunaflux_fp8_act_quant_bytes(int64_t max_rows, int64_t columns) {
  if (max_rows <= 0 || columns <= 0 || max_rows > kMaxDim || columns > kMaxDim) return -1;
  return align_up(max_rows * columns, 256) + align_up(max_rows * 4, 256);
}

static int64_t w8a16_workspace(int32_t entry, int64_t n, int64_t k, int64_t nq, int64_t nkv,
                               int32_t max_tokens) {
  if (w8a16_b128_entry(entry)) {
    W8a16Split sp;
    if (n <= 0 || k <= 0 || max_tokens <= 0 || n > kMaxDim || k > kMaxDim ||
        !w8a16_b128_split(n, k, max_tokens, &sp)) {
      return -1;
    }
    W8a16Gemm gm;
    if (w8a16_gemm(w8a16_channel_entry(entry), n, k, max_tokens, &gm, true)) return w8a16_gemm_workspace(gm);
    if (const W8a16Fixed *f = w8a16_fixed(entry, n, k, nq, nkv, max_tokens)) {
      return w8a16_fixed_workspace(*f, n);
    }
    const int64_t nw = entry == LF_FP8_ENTRY_W8A16_GATE_UP_B128 ? 2 : 1;
    int64_t need = sp.split == 1 ? 256
                                 : align_up(sp.split * (n / 16) * nw * sp.mt * 1024, 256) +
                                       align_up(sp.groups * 4, 256);
    // QKV without its Q / K-V split: also room for the workspace of any
    // specialized entry of this width (the geometry, given the split, may
    // pick one)
    if (entry == LF_FP8_ENTRY_W8A16_QKV_B128 && nq == 0) {
      for (const W8a16Fixed &f : kW8a16Fixed) {
        if (f.entry == entry && n == f.nq + 2 * f.nkv &&
            w8a16_fixed(entry, n, k, f.nq, f.nkv, max_tokens) == &f) {
          need = std::max(need, w8a16_fixed_workspace(f, n));
        }
      }
    }
    return need;
  }
  if (entry != LF_FP8_ENTRY_W8A16_DENSE && entry != LF_FP8_ENTRY_W8A16_QKV &&
      entry != LF_FP8_ENTRY_W8A16_GATE_UP) {
    return -1;
  }
  W8a16Split sp;
  if (n <= 0 || k <= 0 || k % 128 != 0 || max_tokens <= 0 || n > kMaxDim || k > kMaxDim ||
      !w8a16_split(n, k, max_tokens, &sp)) {
    return -1;
  }
  W8a16Gemm gm;
  if (w8a16_gemm(entry, n, k, max_tokens, &gm)) return w8a16_gemm_workspace(gm);
  if (const W8a16Fixed *f = w8a16_fixed(entry, n, k, nq, nkv, max_tokens)) {
    return w8a16_fixed_workspace(*f, n);
  }
  if (sp.split == 1) return 256;
  // One 1 KiB fp32 accumulator fragment per (slice, 16-column tile, weight,
  // 16-row tile), then one arrival counter per column group.
  const int64_t nw = entry == LF_FP8_ENTRY_W8A16_GATE_UP ? 2 : 1;
  return align_up(sp.split * (n / 16) * nw * sp.mt * 1024, 256) + align_up(sp.groups * 4, 256);
}

int64_t lunaflux_fp8_w8a16_workspace_bytes(int32_t entry, int64_t n, int64_t k,
                                           int32_t max_tokens) {
  return w8a16_workspace(entry, n, k, 0, 0, max_tokens);
}

int64_t lunaflux_fp8_gated_mlp_workspace_bytes(int32_t entry, int64_t hidden, int64_t inter,
                                               int32_t max_tokens) {
  if (entry == LF_FP8_ENTRY_W8A8_GATED_MLP_B128) {
    W8a8B128 g;
    if (hidden > kMaxDim || inter > kMaxDim || !w8a8_b128_gated(hidden, inter, max_tokens, &g)) return -1;
    const int64_t cap = g.bands * g.bm;
    return sync_bytes(3, g.bands) + b128_rows_bytes(cap, hidden) + align_up(cap * inter * 2, 256) +
           b128_rows_bytes(cap, inter);
  }
  if (entry == LF_FP8_ENTRY_W8A8_GATED_MLP) {
    W8a8Gated g;
    if (hidden <= 0 || inter <= 0 || max_tokens <= 0 || hidden > kMaxDim || inter > kMaxDim ||
        hidden % 128 != 0 || !w8a8_gated(hidden, inter, max_tokens, &g)) {
      return -1;
    }
    return w8a8_gated_workspace(g, hidden, inter);
  }
  W8a16GatedGemm gg;
  if (hidden > 0 && inter > 0 && hidden <= kMaxDim && inter <= kMaxDim && hidden % 128 == 0 &&
      inter % 128 == 0 && w8a16_gated_gemm(entry, hidden, inter, max_tokens, &gg)) {
    return w8a16_gated_gemm_workspace(gg, inter);
  }
  const W8a16Gated *g = w8a16_gated(entry, hidden, inter, max_tokens);
  return g == nullptr ? -1 : w8a16_gated_workspace(*g);
}

int64_t lunaflux_fp8_w8a8_workspace_bytes(int32_t entry, int64_t n, int64_t k, int32_t max_tokens) {
  if (w8a8_b128_entry(entry)) {
    W8a8B128 t;
    if (n > kMaxDim || k > kMaxDim ||
        !w8a8_b128_tiles(entry == LF_FP8_ENTRY_W8A8_GATE_UP_B128, n, k, max_tokens, &t)) {
      return -1;
    }
    return sync_bytes(1, t.bands) + b128_rows_bytes(t.bands * t.bm, k);
  }
  if ((entry != LF_FP8_ENTRY_W8A8_DENSE_AQ && entry != LF_FP8_ENTRY_W8A8_QKV_AQ &&
       entry != LF_FP8_ENTRY_W8A8_GATE_UP_AQ) ||
      n <= 0 || k <= 0 || k % 128 != 0 || max_tokens <= 0 || n > kMaxDim || k > kMaxDim) {
    return -1;
  }
  W8a8Tiles t;
  if (!w8a8_tiles(entry == LF_FP8_ENTRY_W8A8_GATE_UP_AQ, n, k, max_tokens, &t)) return -1;
  return sync_bytes(1, t.bands) + quantized_rows_bytes(t.bands * t.bm, k);
}

int32_t lunaflux_fp8_gated_mlp_geometry(int32_t entry, int64_t hidden, int64_t inter,
                                        int32_t max_tokens, int32_t dims[7],
                                        char symbol[LF_FP8_SYMBOL_BYTES]) {
  if (dims == nullptr || symbol == nullptr || hidden <= 0 || inter <= 0 || max_tokens <= 0) {
    return LF_INVALID_ARGUMENT;
  }
  if (entry == LF_FP8_ENTRY_W8A8_GATED_MLP_B128) {
    W8a8B128 g;
    if (hidden > kMaxDim || inter > kMaxDim || !w8a8_b128_gated(hidden, inter, max_tokens, &g)) {
      return LF_INVALID_ARGUMENT;
    }
    // x quantizer, gate/up tiles (bm / 2 h-columns each), h quantizer, down
    // tiles
    const int64_t blocks = 2 * kQuantBlocks + g.gx * g.bands;
    if (blocks > INT32_MAX) return LF_INVALID_ARGUMENT;
    const int32_t values[7] = {static_cast<int32_t>(blocks), 1, 1, g.form != 0 ? 512 : 256, 1, 1, 0};
    std::memcpy(dims, values, sizeof(values));
    std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
    std::snprintf(symbol, LF_FP8_SYMBOL_BYTES, "lf_fp8_w8a8_gated_mlp_b128%s", w8a8_b128_suffix(g.form));
    return LF_OK;
  }
  if (entry == LF_FP8_ENTRY_W8A8_GATED_MLP) {
    W8a8Gated g;
    if (hidden > kMaxDim || inter > kMaxDim || hidden % 128 != 0 || inter % 128 != 0 ||
        !w8a8_gated(hidden, inter, max_tokens, &g)) {
      return LF_INVALID_ARGUMENT;
    }
    // x quantizer, gate/up tiles, h quantizer, down tiles
    const int64_t blocks = 2 * kQuantBlocks + (g.gu.gx + g.dn.gx) * g.gu.bands;
    if (blocks > INT32_MAX) return LF_INVALID_ARGUMENT;
    const int32_t values[7] = {static_cast<int32_t>(blocks), 1, 1, g.gu.threads, 1, 1, 0};
    std::memcpy(dims, values, sizeof(values));
    std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
    std::snprintf(symbol, LF_FP8_SYMBOL_BYTES, "lf_fp8_w8a8_gated_mlp_%s_%s", w8a8_form_name(g.gu.form),
                  w8a8_form_name(g.dn.form));
    return LF_OK;
  }
  W8a16GatedGemm gg;
  if (hidden <= kMaxDim && inter <= kMaxDim && hidden % 128 == 0 && inter % 128 == 0 &&
      w8a16_gated_gemm(entry, hidden, inter, max_tokens, &gg)) {
    const int64_t blocks = gg.gu.blocks_n + gg.dn.blocks_n * gg.dn.split;
    if (blocks > INT32_MAX) return LF_INVALID_ARGUMENT;
    const int32_t values[7] = {static_cast<int32_t>(blocks), 1, 1, 512, 1, 1, 0};
    std::memcpy(dims, values, sizeof(values));
    std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
    std::snprintf(symbol, LF_FP8_SYMBOL_BYTES, "lf_fp8_w8a16_gated_mlp%s_m128_n128_n%d",
                  entry == LF_FP8_ENTRY_W8A16_GATED_MLP_B128 ? "_b128" : "", gg.dn.bn);
    return LF_OK;
  }
  const W8a16Gated *g = w8a16_gated(entry, hidden, inter, max_tokens);
  if (g == nullptr) return LF_UNSUPPORTED;
  // gate/up blocks (I / 16 / waves, split 1) then down blocks (H / 16 /
  // waves column groups x the down split)
  const int64_t blocks = g->inter / 16 / g->waves + g->hidden / 16 / g->waves * g->down_split;
  const int32_t values[7] = {static_cast<int32_t>(blocks), 1, 1, 64 * g->waves, 1, 1, 0};
  std::memcpy(dims, values, sizeof(values));
  std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
  std::snprintf(symbol, LF_FP8_SYMBOL_BYTES, "%s", g->symbol);
  return LF_OK;
}

int32_t lunaflux_fp8_rms_norm_quant_geometry(float epsilon, int64_t k, int32_t max_rows,
                                             int32_t dims[7], char symbol[LF_FP8_SYMBOL_BYTES]) {
  if (dims == nullptr || symbol == nullptr || k <= 0 || k > 8192 || k % 128 != 0 ||
      max_rows <= 0) {
    return LF_INVALID_ARGUMENT;
  }
  const char *name = nullptr;
  if (epsilon == 1e-5f) {
    name = "lf_fp8_rms_norm_quant_rows_eps1em5";
  } else if (epsilon == 1e-6f) {
    name = "lf_fp8_rms_norm_quant_rows_eps1em6";
  } else {
    return LF_UNSUPPORTED;
  }
  const int32_t values[7] = {(max_rows + 3) / 4, 1, 1, 256, 1, 1, 0};  // one wave per row
  std::memcpy(dims, values, sizeof(values));
  std::snprintf(symbol, LF_FP8_SYMBOL_BYTES, "%s", name);
  return LF_OK;
}

int64_t lunaflux_fp8_qkv_w8a16_workspace_bytes(int64_t nq, int64_t nkv, int64_t k,
                                               int32_t max_tokens) {
  if (nq <= 0 || nkv <= 0 || nq > kMaxDim || nkv > kMaxDim) return -1;
  return w8a16_workspace(LF_FP8_ENTRY_W8A16_QKV, nq + 2 * nkv, k, nq, nkv, max_tokens);
}

static int32_t launch_geometry(int32_t entry, int64_t n, int64_t k, int64_t nq, int64_t nkv,
                               int32_t max_tokens, int32_t dims[7],
                               char symbol[LF_FP8_SYMBOL_BYTES]) {
  if (dims == nullptr || symbol == nullptr || n <= 0 || k <= 0 ||
      max_tokens <= 0 || n > kMaxDim || k > kMaxDim || k % 128 != 0) {
    return LF_INVALID_ARGUMENT;
  }
  int32_t gx = 1, gy = 1, bx = 256;
  const char *name = nullptr;
  char buffer[LF_FP8_SYMBOL_BYTES];
  switch (entry) {
    case LF_FP8_ENTRY_RMS_NORM_QUANT_ROWS:
      return LF_INVALID_ARGUMENT;  // needs the epsilon: lunaflux_fp8_rms_norm_quant_geometry
    case LF_FP8_ENTRY_ACT_QUANT_ROWS:
      name = "lf_fp8_act_quant_rows";  // one wave per row
      gx = (max_tokens + 3) / 4;
      bx = 256;
      break;
    case LF_FP8_ENTRY_W8A16_DENSE:
    case LF_FP8_ENTRY_W8A16_QKV:
    case LF_FP8_ENTRY_W8A16_GATE_UP: {
      W8a16Split sp;
      if (!w8a16_split(n, k, max_tokens, &sp)) return LF_INVALID_ARGUMENT;
      const char *op = entry == LF_FP8_ENTRY_W8A16_DENSE ? "dense"
                       : entry == LF_FP8_ENTRY_W8A16_QKV ? "qkv"
                                                         : "gate_up";
      W8a16Gemm gm;
      if (w8a16_gemm(entry, n, k, max_tokens, &gm)) {
        std::snprintf(buffer, sizeof(buffer), "lf_fp8_w8a16_%s_m128_n%d", op, gm.bn);
        name = buffer;
        gx = static_cast<int32_t>(gm.blocks_n * gm.split);
        bx = 512;
        break;
      }
      if (const W8a16Fixed *f = w8a16_fixed(entry, n, k, nq, nkv, max_tokens)) {
        name = f->symbol;
        w8a16_fixed_geometry(*f, n, &gx, &bx);
        break;
      }
      std::snprintf(buffer, sizeof(buffer), "lf_fp8_w8a16_%s_m%d%s", op, 16 * sp.mt,
                    sp.one_tile ? "_t1" : "");
      name = buffer;
      gx = static_cast<int32_t>(sp.groups * sp.split);
      bx = 64 * (sp.one_tile ? kW16TileWaves : kW16Waves);
      break;
    }
    case LF_FP8_ENTRY_W8A16_DENSE_B128:
    case LF_FP8_ENTRY_W8A16_QKV_B128:
    case LF_FP8_ENTRY_W8A16_GATE_UP_B128: {
      W8a16Split sp;
      if (!w8a16_b128_split(n, k, max_tokens, &sp)) return LF_INVALID_ARGUMENT;
      const char *op = entry == LF_FP8_ENTRY_W8A16_DENSE_B128 ? "dense"
                       : entry == LF_FP8_ENTRY_W8A16_QKV_B128 ? "qkv"
                                                              : "gate_up";
      W8a16Gemm gm;
      if (w8a16_gemm(w8a16_channel_entry(entry), n, k, max_tokens, &gm, true)) {
        std::snprintf(buffer, sizeof(buffer), "lf_fp8_w8a16_%s_b128_m128_n%d", op, gm.bn);
        name = buffer;
        gx = static_cast<int32_t>(gm.blocks_n * gm.split);
        bx = 512;
        break;
      }
      if (const W8a16Fixed *f = w8a16_fixed(entry, n, k, nq, nkv, max_tokens)) {
        name = f->symbol;
        w8a16_fixed_geometry(*f, n, &gx, &bx);
        break;
      }
      std::snprintf(buffer, sizeof(buffer), "lf_fp8_w8a16_%s_b128_m%d", op, 16 * sp.mt);
      name = buffer;
      gx = static_cast<int32_t>(sp.groups * sp.split);
      bx = 64 * kW16Waves;
      break;
    }
    case LF_FP8_ENTRY_W8A8_DENSE_B128:
    case LF_FP8_ENTRY_W8A8_QKV_B128:
    case LF_FP8_ENTRY_W8A8_GATE_UP_B128: {
      const bool gate_up = entry == LF_FP8_ENTRY_W8A8_GATE_UP_B128;
      W8a8B128 t;
      if (!w8a8_b128_tiles(gate_up, n, k, max_tokens, &t)) return LF_INVALID_ARGUMENT;
      const int64_t blocks = kQuantBlocks + t.gx * t.bands;
      if (blocks > INT32_MAX) return LF_INVALID_ARGUMENT;
      std::snprintf(buffer, sizeof(buffer), "lf_fp8_w8a8_%s_b128%s",
                    entry == LF_FP8_ENTRY_W8A8_QKV_B128 ? "qkv" : gate_up ? "gate_up" : "dense",
                    w8a8_b128_suffix(t.form));
      name = buffer;
      gx = static_cast<int32_t>(blocks);
      bx = t.form != 0 ? 512 : 256;
      break;
    }
    case LF_FP8_ENTRY_W8A8_DENSE:
    case LF_FP8_ENTRY_W8A8_QKV:
    case LF_FP8_ENTRY_W8A8_GATE_UP:
    case LF_FP8_ENTRY_W8A8_DENSE_AQ:
    case LF_FP8_ENTRY_W8A8_QKV_AQ:
    case LF_FP8_ENTRY_W8A8_GATE_UP_AQ: {
      const bool aq = entry == LF_FP8_ENTRY_W8A8_DENSE_AQ || entry == LF_FP8_ENTRY_W8A8_QKV_AQ ||
                      entry == LF_FP8_ENTRY_W8A8_GATE_UP_AQ;
      const bool gate_up = entry == LF_FP8_ENTRY_W8A8_GATE_UP || entry == LF_FP8_ENTRY_W8A8_GATE_UP_AQ;
      const bool qkv = entry == LF_FP8_ENTRY_W8A8_QKV || entry == LF_FP8_ENTRY_W8A8_QKV_AQ;
      W8a8Tiles t;
      if (!w8a8_tiles(gate_up, n, k, max_tokens, &t)) return LF_INVALID_ARGUMENT;
      const int64_t blocks = t.gx * t.bands + (aq ? kQuantBlocks : 0);
      if (blocks > INT32_MAX) return LF_INVALID_ARGUMENT;
      std::snprintf(buffer, sizeof(buffer), "lf_fp8_w8a8_%s_%s%s", qkv ? "qkv" : gate_up ? "gate_up" : "dense",
                    w8a8_form_name(t.form), aq ? "_aq" : "");
      name = buffer;
      gx = static_cast<int32_t>(blocks);
      gy = 1;
      bx = t.threads;
      break;
    }
    default:
      return LF_INVALID_ARGUMENT;
  }
  if (gy > LF_MAX_GRID_YZ) return LF_INVALID_ARGUMENT;
  dims[0] = gx;
  dims[1] = gy;
  dims[2] = 1;
  dims[3] = bx;
  dims[4] = 1;
  dims[5] = 1;
  dims[6] = 0;
  std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
  std::strncpy(symbol, name, LF_FP8_SYMBOL_BYTES - 1);
  return LF_OK;
}

int32_t lunaflux_fp8_launch_geometry(int32_t entry, int64_t n, int64_t k,
                                     int32_t max_tokens, int32_t dims[7],
                                     char symbol[LF_FP8_SYMBOL_BYTES]) {
  return launch_geometry(entry, n, k, 0, 0, max_tokens, dims, symbol);
}

int32_t lunaflux_fp8_qkv_launch_geometry(int32_t entry, int64_t nq, int64_t nkv, int64_t k,
                                         int32_t max_tokens, int32_t dims[7],
                                         char symbol[LF_FP8_SYMBOL_BYTES]) {
  if ((entry != LF_FP8_ENTRY_W8A16_QKV && entry != LF_FP8_ENTRY_W8A8_QKV &&
       entry != LF_FP8_ENTRY_W8A8_QKV_AQ && entry != LF_FP8_ENTRY_W8A16_QKV_B128 &&
       entry != LF_FP8_ENTRY_W8A8_QKV_B128) || nq <= 0 ||
      nkv <= 0 || nq > kMaxDim || nkv > kMaxDim) {
    return LF_INVALID_ARGUMENT;
  }
  // block-scaled QKV: every region's 128-row blocks start on a 128-column
  // boundary of the packed output
  if ((entry == LF_FP8_ENTRY_W8A16_QKV_B128 || entry == LF_FP8_ENTRY_W8A8_QKV_B128) &&
      (nq % 128 != 0 || nkv % 128 != 0)) {
    return LF_INVALID_ARGUMENT;
  }
  return launch_geometry(entry, nq + 2 * nkv, k, nq, nkv, max_tokens, dims, symbol);
}

// Blocks (4 waves, 4 groups per wave per step) for a per-128-group quantizer
// of `groups` groups: at most 1024 blocks, each wave then loops.
static int64_t group_quant_blocks(int64_t groups) {
  const int64_t blocks = (groups + 15) / 16;
  return blocks < 1024 ? blocks : 1024;
}

static bool moe_desc_ok(const lf_fp8_moe_desc *d) {
  return d != nullptr && d->magic == LF_FP8_MOE_MAGIC && d->experts >= 1 && d->experts <= 256 &&
         d->top_k >= 1 && d->top_k <= d->experts && d->top_k <= 16 &&
         (d->route_mode == 0 || d->route_mode == 1) && d->hidden > 0 && d->inter > 0 &&
         d->hidden % 128 == 0 && d->inter % 128 == 0 &&
         (d->group == 0 || (d->group == 128 && d->hidden <= 4096 && d->inter <= 4096));
}

int32_t lunaflux_fp8_moe_descriptor(int32_t experts, int32_t top_k, int32_t route_mode,
                                    int64_t hidden, int64_t inter, int32_t group,
                                    lf_fp8_moe_desc *out) {
  if (out == nullptr || hidden > kMaxDim || inter > kMaxDim) return LF_INVALID_ARGUMENT;
  lf_fp8_moe_desc d;
  std::memset(&d, 0, sizeof(d));
  d.magic = LF_FP8_MOE_MAGIC;
  d.experts = experts;
  d.top_k = top_k;
  d.route_mode = route_mode;
  d.hidden = static_cast<int32_t>(hidden);
  d.inter = static_cast<int32_t>(inter);
  d.group = group;
  if (!moe_desc_ok(&d)) return LF_INVALID_ARGUMENT;
  *out = d;
  return LF_OK;
}

// Mirrors MoeLayout in csrc/kernels/moe.hip.
int32_t lunaflux_fp8_moe_workspace_layout(const lf_fp8_moe_desc *d, int32_t tokens,
                                          int64_t offsets[13]) {
  if (!moe_desc_ok(d) || tokens < 0 || offsets == nullptr) return LF_INVALID_ARGUMENT;
  const int64_t T = tokens, A = T * d->top_k, H = d->hidden, I = d->inter;
  const int64_t gx = d->group > 0 ? H / d->group : 1, gh = d->group > 0 ? I / d->group : 1;
  const int64_t sizes[12] = {
      A * 4,                  // top-k expert ids
      A * 4,                  // top-k weights
      A * 4,                  // sorted assignments
      A * 4,                  // position of each assignment
      (d->experts + 1) * 4,   // expert row offsets
      (3 * d->experts + 3) * 4,  // 128-row, 256-row tile offsets; live expert count, ids
      T * H,                  // quantized tokens
      T * gx * 4,             // token scales
      A * I * 2,              // h (bf16)
      A * I,                  // quantized h
      A * gh * 4,             // h scales
      // y (fp32); before the down GEMM it holds the sort's [chunks][E]
      // int32 count table (chunks of 1024 assignments), so it is never smaller
      std::max<int64_t>(A * H * 4, (A + 1023) / 1024 * d->experts * 4),
  };
  int64_t o = 0;
  for (int i = 0; i < 12; ++i) {
    offsets[i] = o;
    o = align_up(o + sizes[i], 256);
  }
  offsets[12] = o;
  return LF_OK;
}

// Per-channel profiles whose GEMMs run on 256-row tiles take the hidden
// quantizer into the down launch (lf_moe_down_t256_aq); the same condition
// as in lunaflux_fp8_moe_launch_geometry.
static bool moe_tiles256(const lf_fp8_moe_desc *d, int64_t T) {
  const int64_t A = T * d->top_k;
  const bool b128 = d->group == 128;
  return A >= 256 * static_cast<int64_t>(d->experts) && d->inter % 128 == 0 && d->hidden % 256 == 0 &&
         (!b128 || (d->hidden <= 3072 && d->inter <= 3072)) &&
         A * std::max<int64_t>(d->hidden, d->inter) < (int64_t(1) << 32);
}
static bool moe_gemv(const lf_fp8_moe_desc *d, int64_t T) {
  return T <= 32 && d->inter % 64 == 0 && d->hidden % 64 == 0;
}
static bool moe_down_aq(const lf_fp8_moe_desc *d, int64_t T) {
  return d->group == 0 && moe_tiles256(d, T) && !moe_gemv(d, T);
}
// Its counter area (kernels/phases.h): error word, done counter, one 128-byte
// line per 256-row tile of the profile (at most A / 256 + E).
static int64_t moe_sync_bytes(const lf_fp8_moe_desc *d, int64_t T) {
  return moe_down_aq(d, T) ? 256 + 128 * (T * d->top_k / 256 + d->experts + 1) : 0;
}

int64_t lunaflux_fp8_moe_workspace_bytes(const lf_fp8_moe_desc *d, int32_t max_tokens) {
  int64_t offsets[13];
  if (max_tokens <= 0 || lunaflux_fp8_moe_workspace_layout(d, max_tokens, offsets) != LF_OK) {
    return -1;
  }
  return offsets[12] + align_up(moe_sync_bytes(d, max_tokens), 256);
}

int64_t lunaflux_fp8_moe_sync_offset(const lf_fp8_moe_desc *d, int32_t max_tokens) {
  int64_t offsets[13];
  if (max_tokens <= 0 || lunaflux_fp8_moe_workspace_layout(d, max_tokens, offsets) != LF_OK ||
      !moe_down_aq(d, max_tokens)) {
    return -1;
  }
  return offsets[12];
}

int32_t lunaflux_fp8_moe_launch_geometry(int32_t entry, const lf_fp8_moe_desc *d,
                                         int32_t max_tokens, int32_t dims[7],
                                         char symbol[LF_FP8_SYMBOL_BYTES]) {
  if (!moe_desc_ok(d) || max_tokens <= 0 || dims == nullptr || symbol == nullptr) {
    return LF_INVALID_ARGUMENT;
  }
  const int64_t T = max_tokens, A = T * d->top_k;
  // Upper bound on the 128-row tiles over all experts: each expert adds at
  // most one partial tile.
  const int64_t tiles = A / 128 + d->experts;
  const bool b128 = d->group == 128;
  // Profiles averaging >= 256 routed rows per expert run the
  // grouped GEMMs on 256 x 256 tiles (8 waves; each weight strip streamed
  // once per 256 rows), smaller ones on 128 x 128 tiles.
  // Block-scaled profiles too, for K <= 3072 in both GEMMs (their row-ratio
  // table shares the LDS with the stage ring).
  // Their activation rows are addressed by 32-bit offsets into the token
  // and assignment arrays: A rows x max(H, I) < 2^32.
  const bool t256 = moe_tiles256(d, T);
  const int64_t tiles256 = A / 256 + d->experts;
  // Profiles of at most 32 tokens (every expert <= 32 rows) run the grouped
  // GEMV form: a fixed grid (up to 4 blocks per CU) whose blocks loop over
  // the (expert with rows, 4 consecutive 16-column tiles) items.
  const bool gemv = moe_gemv(d, T);
  // per-channel 256-row tiles: the hidden quantizer is the down launch's
  // first step (kQuantBlocks blocks ahead of its tiles)
  const bool down_aq = moe_down_aq(d, T);
  const int64_t kGemvBlocks = 1024;
  int64_t gx = 1, gy = 1;
  int32_t bx = 256;
  const char *name = nullptr;
  switch (entry) {
    // Routing and the per-token quantizers: one wave per token (row); the
    // per-128-column-group quantizers: four groups per wave.
    // Profiles of at most 1024 assignments route, sort and quantize the
    // tokens in one launch (lf_moe_route_sort, one 1024-thread block); the
    // two sort steps and the token quantizer then launch nothing (empty
    // symbol, zero dims).
    case LF_FP8_MOE_ROUTE:
      if (A <= 1024) {
        name = "lf_moe_route_sort";
        bx = 1024;
        break;
      }
      name = "lf_moe_route";
      gx = (T + 3) / 4;
      break;
    // The sort: one 1024-thread block per chunk of 1024 assignments.
    case LF_FP8_MOE_SORT_COUNT:
    case LF_FP8_MOE_SORT:
      if (A <= 1024) {
        std::memset(dims, 0, 7 * sizeof(int32_t));
        std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
        return LF_OK;
      }
      name = entry == LF_FP8_MOE_SORT ? "lf_moe_sort" : "lf_moe_sort_count";
      gx = (A + 1023) / 1024;
      bx = 1024;
      break;
    case LF_FP8_MOE_QUANT_TOKENS:
      if (A <= 1024) {  // quantized by lf_moe_route_sort
        std::memset(dims, 0, 7 * sizeof(int32_t));
        std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
        return LF_OK;
      }
      name = "lf_moe_quant_tokens";
      gx = b128 ? group_quant_blocks(T * (d->hidden / 128)) : (T + 3) / 4;
      break;
    case LF_FP8_MOE_GATE_UP:
      if (gemv) {
        name = "lf_moe_gate_up_gemv";
        gx = std::min<int64_t>(std::min<int64_t>(d->experts, A) * (d->inter / 64), kGemvBlocks);
        break;
      }
      // 1-D grid over (64 h-column block, 128-row tile); blocks past the
      // live tile count return.
      // (block scales: the epilogue also quantizes h, see QUANT_HIDDEN)
      if (t256) {
        name = b128 ? "lf_moe_gate_up_t256_b128_q" : "lf_moe_gate_up_t256";
        gx = d->inter / 128 * tiles256;
        bx = 512;
        break;
      }
      name = b128 ? "lf_moe_gate_up_b128" : "lf_moe_gate_up";
      gx = d->inter / 64 * tiles;
      break;
    case LF_FP8_MOE_QUANT_HIDDEN:
      if ((t256 && b128 && !gemv) || down_aq) {
        // fused into the gate/up epilogue (block scales) or run as the down
        // launch's first step (per-token): no launch (empty symbol, zero dims)
        std::memset(dims, 0, 7 * sizeof(int32_t));
        std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
        return LF_OK;
      }
      name = "lf_moe_quant_hidden";
      gx = b128 ? group_quant_blocks(A * (d->inter / 128)) : (A + 3) / 4;
      break;
    case LF_FP8_MOE_DOWN:
      if (gemv) {
        name = "lf_moe_down_gemv";
        gx = std::min<int64_t>(std::min<int64_t>(d->experts, A) * (d->hidden / 64), kGemvBlocks);
        break;
      }
      if (t256) {
        name = b128 ? "lf_moe_down_t256_b128" : "lf_moe_down_t256_aq";
        gx = d->hidden / 256 * tiles256 + (down_aq ? kQuantBlocks : 0);
        bx = 512;
        break;
      }
      name = b128 ? "lf_moe_down_b128" : "lf_moe_down";
      gx = d->hidden / 128 * tiles;
      break;
    case LF_FP8_MOE_COMBINE: name = "lf_moe_combine"; gx = T; break;
    default: return LF_INVALID_ARGUMENT;
  }
  if (gx > INT32_MAX || gy > LF_MAX_GRID_YZ) return LF_INVALID_ARGUMENT;
  dims[0] = static_cast<int32_t>(gx);
  dims[1] = static_cast<int32_t>(gy);
  dims[2] = 1;
  dims[3] = bx;
  dims[4] = 1;
  dims[5] = 1;
  dims[6] = 0;
  std::memset(symbol, 0, LF_FP8_SYMBOL_BYTES);
  std::strncpy(symbol, name, LF_FP8_SYMBOL_BYTES - 1);
  return LF_OK;
}

}  // extern "C"
