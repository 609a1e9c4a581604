// moe.hip - the grouped (expert MLP) form of the FP8 projection path.
//
// Launch sequence of one MoE expert-MLP operation (all operands are device
// regions; `desc` is the routing descriptor, `ws` the operation's workspace,
// whose layout is a function of the live token count T and the descriptor,
// recomputed identically by every kernel - see MoeLayout):
//   lf_moe_route          logits [T, E] fp32       -> top-k experts, weights
//   lf_moe_sort_count     per-chunk expert counts of the T*k assignments
//   lf_moe_sort           stable counting sort of the assignments by expert
//                         -> sorted ids, positions, per-expert row offsets
//                         and 128-row tile offsets
//   lf_moe_quant_tokens   x [T, H] bf16            -> e4m3 + scales (per token
//                         or per token per 128 columns)
//   lf_moe_gate_up        grouped GEMM over expert gate/up weights with the
//                         gathered token rows, SwiGLU epilogue -> h [T*k, I]
//                         bf16 in expert order
//   lf_moe_quant_hidden   h -> e4m3 + scales
//   lf_moe_down           grouped GEMM over expert down weights -> y [T*k, H]
//                         bf16 in expert order
//   lf_moe_combine        out[t] = sum_j w[t, j] * y[pos(t, j)] (j ascending)
//                         -> bf16 [T, H]
#include "w8a8_core.h"
#include "w8a8_v3.h"
#include "w8a8_v4.h"

namespace {

constexpr uint32_t kMoeMagic = 0x454F4D4Cu;  // bytes "LMOE"

struct MoeDesc {
  uint32_t magic;
  int32_t experts, top_k, route_mode, hidden, inter, group, reserved;
};

LF_DEVICE uint64_t al256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

// Byte offsets of the workspace arrays for T live tokens (mirrored on the
// host by lunaflux_fp8_moe_workspace_bytes).
struct MoeLayout {
  uint64_t topk_ids, topk_w, sorted, pos, offsets, tiles, xq, xs, h, hq, hs, y, end;
  LF_DEVICE MoeLayout(const MoeDesc &d, int T) {
    const uint64_t A = static_cast<uint64_t>(T) * d.top_k;
    const uint64_t H = d.hidden, I = d.inter;
    const uint64_t gx = d.group > 0 ? H / d.group : 1, gh = d.group > 0 ? I / d.group : 1;
    uint64_t o = 0;
    topk_ids = o; o = al256(o + A * 4);
    topk_w = o;   o = al256(o + A * 4);
    sorted = o;   o = al256(o + A * 4);
    pos = o;      o = al256(o + A * 4);
    offsets = o;  o = al256(o + (d.experts + 1) * 4);
    // 128-row tile prefix [E + 1], the 256-row tile prefix [E + 1], the
    // number of experts with rows, then their ids ascending [E]
    tiles = o;    o = al256(o + (3 * d.experts + 3) * 4);
    xq = o;       o = al256(o + static_cast<uint64_t>(T) * H);
    xs = o;       o = al256(o + static_cast<uint64_t>(T) * gx * 4);
    h = o;        o = al256(o + A * I * 2);
    hq = o;       o = al256(o + A * I);
    hs = o;       o = al256(o + A * gh * 4);
    // y also holds the sort's [chunks][E] count table before the down GEMM
    const uint64_t table = ((A + 1023) / 1024) * d.experts * 4;
    y = o;        o = al256(o + (A * H * 4 > table ? A * H * 4 : table));
    end = o;
  }
};

template <typename T>
LF_DEVICE T *at(uint8_t *ws, uint64_t offset) {
  return reinterpret_cast<T *>(ws + offset);
}

LF_DEVICE bool desc_ok(const MoeDesc &d) {
  return d.magic == kMoeMagic && d.experts > 0 && d.experts <= 256 && d.top_k > 0 &&
         d.top_k <= d.experts && d.top_k <= 16;
}

// --- routing ---------------------------------------------------------------
// One wave per token, four tokens per block; lane l holds the logits of
// experts l, l + 64, ... (E <= 256) and the wave keeps their ranking keys in
// LDS. The k largest logits in order (ties -> lower expert id) by rank: each
// lane counts the keys that beat each of its own, so the expert ranked r < k
// is the r-th pick, with no serial cross-lane chain. A key is one 64-bit
// integer (rank_key64) that orders as the logit and then the lower id does,
// so "beats" is one integer compare (a compare and a carry-add per key; the
// float form, u > v or u == v and j < e, cost boolean mask logic on the
// scalar unit per key: 2.5 us per token at E = 64 against 0.8 us measured).
// Softmax weights over the k picked logits (mode 0) or over all experts (mode
// 1); the sum of exponentials is accumulated in expert order, as the
// reference loop does (every lane reads the exponentials back from LDS and
// sums them in that order).
LF_DEVICE void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The ranking key of a logit: the logit itself, with NaN as -inf. On these
// keys "beats" (u > v, or u == v and a lower id) is a strict total order, so
// the ranks of one token's experts are a permutation of 0 .. E-1 and every
// pick slot r < k is written once, whatever the logits hold. A NaN logit thus
// ranks below every finite one (ties by id); a token whose top key is
// non-finite (+inf, or every logit NaN or -inf) gets NaN weights, and its
// output row comes out NaN. The reference rejects non-finite values
// (kernels/reference/basic.mbt:91-93); a kernel cannot raise, so it keeps
// every index in range and lets the value carry the fault.
LF_DEVICE float rank_key(float v) { return __builtin_isnan(v) ? -__builtin_inff() : v; }

// rank_key as a 64-bit integer with the expert id below it: the key's bits
// mapped to a signed integer in float order (negative floats have their
// magnitude bits flipped; -0 is first made +0, which compares equal to it),
// times 256, plus 255 - e. Key a > key b exactly when a's logit ranks above
// b's or they are equal and a's id is lower. Slots past E hold INT64_MIN,
// below every key.
LF_DEVICE int64_t rank_key64(float v, int e) {
  const int32_t b = __float_as_int(rank_key(v) + 0.0f);
  const int32_t o = b >= 0 ? b : b ^ 0x7fffffff;
  return static_cast<int64_t>(o) * 256 + (255 - e);
}
typedef int64_t i64x2 __attribute__((ext_vector_type(2)));

// This lane's logits of token t (experts lane, lane + 64, lane + 128,
// lane + 192; 0 past E).
struct TokenLogits {
  float v[4];
};
LF_DEVICE TokenLogits route_load(const MoeDesc &d, const float *logits, int t) {
  const int lane = threadIdx.x & 63;
  const int E = d.experts;
  const float *l = logits + static_cast<uint64_t>(t) * E;
  TokenLogits r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    r.v[i] = e < E ? l[e] : 0.0f;
  }
  return r;
}

// Routes token t, whose logits lg holds, with the calling wave; sk (256
// keys, 16-byte aligned), sid and spv (16 each) are this wave's LDS scratch.
LF_DEVICE void route_ranked(const MoeDesc &d, const MoeLayout &L, uint8_t *ws, int t,
                            const TokenLogits &lg, int64_t *sk, int32_t *sid, float *spv) {
  const int lane = threadIdx.x & 63;
  const int E = d.experts, k = d.top_k;
  int32_t *ids = at<int32_t>(ws, L.topk_ids) + static_cast<uint64_t>(t) * k;
  float *wts = at<float>(ws, L.topk_w) + static_cast<uint64_t>(t) * k;
  float v[4];
  int64_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? rank_key(lg.v[i]) : 0.0f;
    key[i] = e < E ? rank_key64(lg.v[i], e) : INT64_MIN;
    sk[e] = key[i];
  }
  wave_lds_sync();
  const int E2 = (E + 1) & ~1;  // an odd E reads the INT64_MIN slot E too
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    if (e >= E) break;
    int r = 0;
#pragma unroll 8
    for (int j = 0; j < E2; j += 2) {
      const i64x2 u = *reinterpret_cast<const i64x2 *>(&sk[j]);
      r += u.x > key[i] ? 1 : 0;
      r += u.y > key[i] ? 1 : 0;
    }
    if (r < k) {
      sid[r] = e;
      spv[r] = v[i];
    }
  }
  wave_lds_sync();
  const float top = spv[0];
  float sum = 0.0f;
  if (d.route_mode == 0) {
    for (int j = 0; j < k; ++j) sum += expf(spv[j] - top);
  } else {
    // the ranking above has read sk for the last time; the exponentials
    // take its first E floats
    float *sv = reinterpret_cast<float *>(sk);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      if (e < E) sv[e] = expf(v[i] - top);
    }
    wave_lds_sync();
    const int E4 = E & ~3;
#pragma unroll 8
    for (int j = 0; j < E4; j += 4) {
      const float4 u = *reinterpret_cast<const float4 *>(&sv[j]);
      sum += u.x;
      sum += u.y;
      sum += u.z;
      sum += u.w;
    }
    for (int j = E4; j < E; ++j) sum += sv[j];
  }
  if (lane < k) {
    ids[lane] = sid[lane];
    wts[lane] = expf(spv[lane] - top) / sum;
  }
  // the next token of this wave overwrites sk, sid and spv
  wave_lds_sync();
}

LF_DEVICE void route_token(const MoeDesc &d, const MoeLayout &L, const float *logits, uint8_t *ws,
                           int t, int64_t *sk, int32_t *sid, float *spv) {
  route_ranked(d, L, ws, t, route_load(d, logits, t), sk, sid, spv);
}

LF_DEVICE void route(const int32_t *counts, const MoeDesc &d, const float *logits, uint8_t *ws) {
  __shared__ __attribute__((aligned(16))) int64_t sk[4][256];
  __shared__ int32_t sid[4][16];
  __shared__ float spv[4][16];
  const int T = live_rows(counts, 1 << 30);
  const int w = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + w;
  if (t >= T) return;
  route_token(d, MoeLayout(d, T), logits, ws, t, sk[w], sid[w], spv[w]);
}

// --- stable counting sort ----------------------------------------------------
// Two launches over chunks of 1024 assignments (one 1024-thread block per
// chunk). lf_moe_sort_count: each block counts its chunk's assignments per
// expert into a [chunks][E] table. lf_moe_sort: each block sums the table
// (expert totals, and the counts of the chunks before its own), derives the
// expert row offsets, and ranks its chunk's assignments among equal experts:
// within a wave by matching expert ids with ballots over their bits, across
// the chunk's waves by a prefix over per-wave counts. Positions therefore
// equal those of a stable sort. The table lives at the start of the y
// region, which nothing reads before the down GEMM overwrites it.
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;

LF_DEVICE int32_t *chunk_table(uint8_t *ws, const MoeLayout &L) { return at<int32_t>(ws, L.y); }

// An expert id read back from the workspace, as both sort kernels use it:
// lf_moe_route writes only ids in [0, E), so this is the identity there; an id
// outside that range (a workspace written by something else) counts as
// expert 0 in both kernels alike, so every assignment still gets exactly one
// position and no count or position index leaves its array.
LF_DEVICE int sort_expert(int32_t id, int E) {
  return static_cast<uint32_t>(id) < static_cast<uint32_t>(E) ? id : 0;
}

LF_DEVICE void sort_count(const int32_t *counts, const MoeDesc &d, uint8_t *ws) {
  __shared__ int32_t cnt[256];
  const int T = live_rows(counts, 1 << 30);
  const MoeLayout L(d, T);
  const int E = d.experts, A = T * d.top_k;
  const int c = blockIdx.x;
  if (c * kSortThreads >= A) return;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += kSortThreads) cnt[e] = 0;
  __syncthreads();
  const int a = c * kSortThreads + tid;
  if (a < A) atomicAdd(&cnt[sort_expert(at<int32_t>(ws, L.topk_ids)[a], E)], 1);
  __syncthreads();
  int32_t *table = chunk_table(ws, L) + static_cast<uint64_t>(c) * E;
  for (int e = tid; e < E; e += kSortThreads) table[e] = cnt[e];
}

// Writes an empty routing result: every expert without rows (the GEMMs then
// launch no tile).
LF_DEVICE void sort_write_empty(const MoeDesc &d, const MoeLayout &L, uint8_t *ws) {
  const int E = d.experts;
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    at<int32_t>(ws, L.offsets)[e] = 0;
    at<int32_t>(ws, L.tiles)[e] = 0;
    at<int32_t>(ws, L.tiles)[E + 1 + e] = 0;
  }
  if (threadIdx.x == 0) at<int32_t>(ws, L.tiles)[2 * E + 2] = 0;  // no expert has rows
}

// Exclusive scans over the experts by wave 0 (lane l holds experts 4l ..
// 4l + 3), from the expert totals in wcnt[0]: first row, first 128-row tile
// and first 256-row tile of each expert, and its index in the list of
// experts with rows; written to the workspace when write_global, and the
// first row added to base[e]. The caller synchronizes the block before and
// after.
LF_DEVICE void sort_scan_experts(const MoeDesc &d, const MoeLayout &L, uint8_t *ws, bool write_global,
                                 int32_t *base, int32_t (*wcnt)[256]) {
  const int E = d.experts;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave != 0) return;
  int32_t *offsets = at<int32_t>(ws, L.offsets);
  int32_t *tiles = at<int32_t>(ws, L.tiles);
  int n4[4], r = 0, t1 = 0, t2 = 0, lv = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * lane + i;
    n4[i] = e < E ? wcnt[0][e] : 0;
    r += n4[i];
    t1 += (n4[i] + w8a8::kBM - 1) / w8a8::kBM;
    t2 += (n4[i] + 2 * w8a8::kBM - 1) / (2 * w8a8::kBM);
    lv += n4[i] > 0 ? 1 : 0;
  }
  int off = r, tl = t1, tl2 = t2, live = lv;  // inclusive scans across lanes
#pragma unroll
  for (int step = 1; step < 64; step <<= 1) {
    const int a0 = __shfl_up(off, step), a1 = __shfl_up(tl, step), a2 = __shfl_up(tl2, step),
              a3 = __shfl_up(live, step);
    if (lane >= step) {
      off += a0;
      tl += a1;
      tl2 += a2;
      live += a3;
    }
  }
  off -= r;
  tl -= t1;
  tl2 -= t2;
  live -= lv;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * lane + i;
    if (e < E) {
      if (write_global) {
        offsets[e] = off;
        tiles[e] = tl;
        tiles[E + 1 + e] = tl2;
        if (n4[i] > 0) tiles[2 * E + 3 + live] = e;
      }
      base[e] += off;
    }
    off += n4[i];
    tl += (n4[i] + w8a8::kBM - 1) / w8a8::kBM;
    tl2 += (n4[i] + 2 * w8a8::kBM - 1) / (2 * w8a8::kBM);
    live += n4[i] > 0 ? 1 : 0;
  }
  if (write_global && lane == 63) {  // experts past E count 0: lane 63 holds the totals
    offsets[E] = off;
    tiles[E] = tl;
    tiles[E + 1 + E] = tl2;
    tiles[2 * E + 2] = live;
  }
}

// Positions of chunk c's assignments (a = c * kSortThreads + thread < A)
// from base[e], the first position of expert e's rows of this chunk: ranks
// among equal experts within a wave by matching expert ids with ballots over
// their bits, across the chunk's waves by a prefix over per-wave counts
// (left in wcnt[wave][e] on return). Every thread of a kSortThreads-thread
// block calls it; it synchronizes the block inside.
LF_DEVICE void sort_rank_chunk(const MoeDesc &d, const MoeLayout &L, uint8_t *ws, int A, int c,
                               const int32_t *base, int32_t (*wcnt)[256]) {
  const int E = d.experts;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t *ids = at<int32_t>(ws, L.topk_ids);
  int32_t *sorted = at<int32_t>(ws, L.sorted);
  int32_t *pos = at<int32_t>(ws, L.pos);
  for (int i = tid; i < kSortWaves * E; i += kSortThreads) wcnt[i / E][i % E] = 0;
  int bits = 0;
  while ((1 << bits) < E + 1) ++bits;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  __syncthreads();
  const int a = c * kSortThreads + tid;
  const int e = a < A ? sort_expert(ids[a], E) : E;  // E marks lanes past the end
  uint64_t same = ~0ull;
  for (int b = 0; b < bits; ++b) {
    const uint64_t ones = __ballot((e >> b) & 1);
    same &= ((e >> b) & 1) ? ones : ~ones;
  }
  const int rank = __popcll(same & lt_mask);
  if (e < E && rank == 0) wcnt[wave][e] = __popcll(same);
  __syncthreads();
  if (e < E) {
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wcnt[w][e];
    const int p = base[e] + before + rank;
    sorted[p] = a;
    pos[a] = p;
  }
}

LF_DEVICE void sort_assignments(const int32_t *counts, const MoeDesc &d, uint8_t *ws) {
  __shared__ int32_t base[256];  // first position of expert e's rows of this chunk
  __shared__ int32_t wcnt[kSortWaves][256];
  const int T = live_rows(counts, 1 << 30);
  const MoeLayout L(d, T);
  const int E = d.experts;
  const int A = T * d.top_k;
  const int c = blockIdx.x;
  if (A == 0) {
    if (c == 0) sort_write_empty(d, L, ws);
    return;
  }
  if (c * kSortThreads >= A) return;
  const int chunks = (A + kSortThreads - 1) / kSortThreads;
  const int tid = threadIdx.x;
  const int32_t *table = chunk_table(ws, L);
  // Per expert: total rows and rows in the chunks before this one, every
  // (chunk, expert) entry of the table loaded by its own thread and added
  // into LDS (integer sums: the order does not matter).
  for (int e = tid; e < E; e += kSortThreads) {
    wcnt[0][e] = 0;
    base[e] = 0;
  }
  __syncthreads();
  for (int i = tid; i < chunks * E; i += kSortThreads) {
    const int cc = i / E, e = i - cc * E;
    const int n = table[i];
    atomicAdd(&wcnt[0][e], n);
    if (cc < c) atomicAdd(&base[e], n);
  }
  __syncthreads();
  sort_scan_experts(d, L, ws, c == 0, base, wcnt);
  __syncthreads();
  sort_rank_chunk(d, L, ws, A, c, base, wcnt);
}

// Routing, the whole sort and the token quantizer in one block of
// kSortThreads threads, for profiles with few assignments (the launch
// geometry picks it when max_tokens * top_k <= kSortThreads, where
// lf_moe_route, lf_moe_sort_count, lf_moe_sort and lf_moe_quant_tokens are
// four launches of a few microseconds each): half of the waves route the
// tokens (route_ranked, as lf_moe_route) while the other half quantize them
// as lf_moe_quant_tokens does (the per-token form with the two-pass row
// quantizer, whose codes and scales equal the register-resident one's: a
// 1024-thread block leaves a wave 128 registers); then the block counts the
// assignments per expert, scans as lf_moe_sort, and ranks the chunks of
// kSortThreads assignments in order, each chunk's positions starting where
// the previous chunk's rows of each expert ended. Outputs equal those of the
// four launches for any number of tokens.
LF_DEVICE void route_sort_block(const int32_t *counts, const MoeDesc &d, const float *logits,
                                const uint16_t *x, uint8_t *ws) {
  __shared__ __attribute__((aligned(16))) int64_t sk[kSortWaves][256];
  __shared__ int32_t sid[kSortWaves][16];
  __shared__ float spv[kSortWaves][16];
  __shared__ int32_t base[256];
  __shared__ int32_t wcnt[kSortWaves][256];
  const int T = live_rows(counts, 1 << 30);
  const MoeLayout L(d, T);
  const int E = d.experts;
  const int A = T * d.top_k;
  const int tid = threadIdx.x, wave = tid >> 6;
  // The first half of the waves routes the tokens while the second half
  // runs the token quantizer (codes and token scales need no routing; the
  // per-token form's expert-order copies of the scales are written after the
  // sort).
  constexpr int kRouteWaves = kSortWaves / 2;
  if (wave < kRouteWaves) {
    // A wave's tokens are taken in batches of 4 whose logits are all loaded
    // before the first is ranked (one load latency per batch, not per token).
    constexpr int kBatch = 4;
    for (int t0 = wave; t0 < T; t0 += kBatch * kRouteWaves) {
      TokenLogits lg[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int t = t0 + b * kRouteWaves;
        lg[b] = route_load(d, logits, t < T ? t : t0);
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int t = t0 + b * kRouteWaves;
        if (t < T) route_ranked(d, L, ws, t, lg[b], sk[wave], sid[wave], spv[wave]);
      }
    }
  } else if (d.group != 0) {
    quantize_groups_wave(x, d.hidden, T, at<uint8_t>(ws, L.xq), at<float>(ws, L.xs), wave - kRouteWaves,
                         kSortWaves - kRouteWaves);
  } else {
    for (int t = wave - kRouteWaves; t < T; t += kSortWaves - kRouteWaves) {
      const uint64_t off = static_cast<uint64_t>(t) * d.hidden;
      quantize_row_wave_2pass(x + off, d.hidden, at<uint8_t>(ws, L.xq) + off, at<float>(ws, L.xs) + t);
    }
  }
  // the ids and token scales written above are visible to the whole block
  // after the barrier
  __syncthreads();
  if (A == 0) {
    sort_write_empty(d, L, ws);
    return;
  }
  for (int e = tid; e < E; e += kSortThreads) {
    wcnt[0][e] = 0;
    base[e] = 0;
  }
  __syncthreads();
  const int32_t *ids = at<int32_t>(ws, L.topk_ids);
  for (int a = tid; a < A; a += kSortThreads) atomicAdd(&wcnt[0][sort_expert(ids[a], E)], 1);
  __syncthreads();
  sort_scan_experts(d, L, ws, true, base, wcnt);
  __syncthreads();
  for (int c = 0; c * kSortThreads < A; ++c) {
    sort_rank_chunk(d, L, ws, A, c, base, wcnt);
    __syncthreads();
    // the next chunk's rows of expert e start after this chunk's
    for (int e = tid; e < E; e += kSortThreads) {
      int n = 0;
      for (int w = 0; w < kSortWaves; ++w) n += wcnt[w][e];
      base[e] += n;
    }
    __syncthreads();
  }
  // Per-token form: each token's scale also goes to its assignments'
  // positions in expert order (the positions written above are visible to
  // the block after the last barrier).
  if (d.group == 0) {
    const float *xs = at<float>(ws, L.xs);
    const int32_t *pos = at<int32_t>(ws, L.pos);
    float *hs = at<float>(ws, L.hs);
    for (int a = tid; a < A; a += kSortThreads) hs[pos[a]] = xs[a / d.top_k];
  }
}

// --- quantizers --------------------------------------------------------------
// Per token (group 0): one wave per row, four rows per block. Per 128-column
// group: 16 lanes per group, four groups per wave at a time, the grid's waves
// striding over all groups.
LF_DEVICE void quant_rows(const uint16_t *src, int K, int group, uint8_t *dst, float *scales,
                           int rows) {
  if (group == 0) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    quantize_row_wave(src + static_cast<uint64_t>(row) * K, K, dst + static_cast<uint64_t>(row) * K,
                      scales + row);
  } else {
    quantize_groups_wave(src, K, rows, dst, scales, blockIdx.x * 4 + (threadIdx.x >> 6),
                         gridDim.x * 4);
  }
}

// --- grouped GEMM -------------------------------------------------------------
// The expert owning row tile j of a tile prefix (tiles[0] = 0, nondecreasing,
// j < tiles[E]), with its first tile and its routed-row range, found by the
// whole block in one round of loads: thread t < E tests tiles[t] <= j <
// tiles[t + 1], which exactly one expert satisfies (an expert without tiles
// has tiles[t] == tiles[t + 1]), and publishes t, tiles[t], offsets[t] and
// offsets[t + 1] in LDS. A binary search instead costs log2(E) dependent
// global loads per block. Every thread of the block calls it (barriers
// inside); E <= blockDim.x. The slots start as expert 0 with no rows, so an
// inconsistent prefix yields an in-range expert and an empty row range.
struct TileExpert {
  int e, first_tile, row_begin, row_end;
};
LF_DEVICE TileExpert find_tile_expert(const int32_t *tiles, const int32_t *offsets, int E, int j) {
  __shared__ int found[4];
  const int t = threadIdx.x;
  if (t == 0) {
    found[0] = 0;
    found[1] = j;
    found[2] = 0;
    found[3] = 0;
  }
  __syncthreads();
  if (t < E) {
    const int lo = tiles[t], hi = tiles[t + 1];
    const int o0 = offsets[t], o1 = offsets[t + 1];
    if (lo <= j && j < hi) {
      found[0] = t;
      found[1] = lo;
      found[2] = o0;
      found[3] = o1;
    }
  }
  __syncthreads();
  return {found[0], found[1], found[2], found[3]};
}

// The grouped GEMMs run the direct-to-LDS main loop (w8a8_v3.h) on 128 x 128
// blocks of 4 waves, two blocks per CU, over a 1-D grid in the XCD-aware
// tile order: tile (bx, by) is column block bx of row tile by, where row
// tiles are the 128-row tiles of all experts (tiles[] prefix). The order is
// column-major over all row tiles (one group): the expert weights (E x N x K
// bytes) dwarf the gathered activations, so each XCD takes a range of
// weight columns and streams every weight strip once, for all row tiles of
// its expert back to back, while the activations stay in L2/MALL.
using GemmTile = w8a8v3::Tile<128, 128, 2, 2, 2>;
static_assert(GemmTile::kWaveM * GemmTile::kWgm == w8a8::kBM, "row tiles of the sort");

// A pointer the compiler can treat as wave-uniform (the caller guarantees it
// is): both halves through readfirstlane.
template <typename P>
LF_DEVICE const P *uniform_ptr(const P *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const P *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Block-scaled fold: each k-tile's products times (activation scale of the
// row, k-group) x (weight scale of the column's 128-block, k-group).
struct BlockScaleFold {
  static constexpr bool kActive = true;
  const float *sa_lds;  // [128][KT]
  int KT, wm, lane;
  const float *sw[GemmTile::kFN];  // slot j: [KT] scales of its 128-column block
  template <class A>
  LF_DEVICE void operator()(int kt, const A &step, A &acc, int live) const {
    float swk[GemmTile::kFN];
#pragma unroll
    for (int j = 0; j < GemmTile::kFN; ++j) swk[j] = sw[j][kt];
#pragma unroll
    for (int i = 0; i < GemmTile::kFM; ++i) {
      if (i >= live) continue;  // a fragment with no live row
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float sa = sa_lds[w8a8v3::acc_row<GemmTile>(wm, i, lane, rr) * KT + kt];
#pragma unroll
        for (int j = 0; j < GemmTile::kFN; ++j) acc[i][j][rr] += step[i][j][rr] * (sa * swk[j]);
      }
    }
  }
};

// STAGE 0: gate/up (x rows gathered by token, SwiGLU, bf16 h): a block
// computes 64 h-columns (wave wn: its kFN / 2 gate tiles, then the up tiles
// of the same columns). STAGE 1: down (h rows in expert order, bf16 y): a
// block computes 128 columns.
template <int STAGE, bool BLOCK>
__device__ __forceinline__ void grouped_gemm(const int32_t *counts, const MoeDesc &d, const uint8_t *w0,
                             const uint8_t *w1, uint8_t *ws) {
  using T = GemmTile;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::kSmem];
  // Block-scaled form: activation scales of the block's rows, [128][KT],
  // K <= 4096 (the host rejects larger K for 128-column groups).
  __shared__ float sa_lds[BLOCK ? 128 * 32 : 1];
  const int Tn = live_rows(counts, 1 << 30);
  if (Tn == 0) return;
  const MoeLayout L(d, Tn);
  const int32_t *tiles = at<int32_t>(ws, L.tiles);
  const int E = d.experts;
  const WeightHeader &h0 = header_of(w0);
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int N = static_cast<int>(h0.rows);
  if (BLOCK && KT > 32) return;  // sa_lds holds at most 32 scale columns
  const int gx = STAGE == 0 ? N / 64 : N / 128;
  int bx, by;
  if (!w8a8v3::tile_of_block(gx, tiles[E], tiles[E], bx, by)) return;
  const TileExpert te = find_tile_expert(tiles, at<int32_t>(ws, L.offsets), E, by);
  const int e = te.e;
  const int p0 = te.row_begin + (by - te.first_tile) * 128;
  const int pend = te.row_end;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;
  const int32_t *sorted = at<int32_t>(ws, L.sorted);
  auto src_row = [&](int p) { return STAGE == 0 ? sorted[p] / d.top_k : p; };

  // Block-local weight tile s (16 columns): region, tile index, column.
  auto slot = [&](int s, const uint8_t *&region, int &col) {
    if (STAGE == 0) {
      const int sw = s / T::kFN, f = s % T::kFN;
      const bool up = f >= T::kFN / 2;
      col = bx * 64 + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN / 2 : f);
      region = up ? w1 : w0;
    } else {
      col = bx * 128 + 16 * s;
      region = w0;
    }
  };

  const uint8_t *abase = at<uint8_t>(ws, STAGE == 0 ? L.xq : L.hq);
  const float *ascales = at<float>(ws, STAGE == 0 ? L.xs : L.hs);
  w8a8v3::Plan<T> plan;
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v3::a_load_row<T>(wave, q, lane);
    const int p = p0 + tr < pend ? p0 + tr : p0;  // dead rows re-read the first row
    plan.a[q] = abase + static_cast<uint64_t>(src_row(p)) * K + w8a8v3::a_load_chunk(tr, lane) * 16;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const int half = w8a8v3::b_load_half<T>(wave, q);
    const uint8_t *region;
    int col;
    slot(half >> 1, region, col);
    plan.b[q] = expert_tiles(region, e) + static_cast<uint64_t>(col >> 4) * KT * kTileBytes +
                (half & 1) * 1024 + lane * 16;
  }
  const float *wsc[T::kFN];
  int col[T::kFN];
#pragma unroll
  for (int j = 0; j < T::kFN; ++j) {
    const uint8_t *region;
    slot(wn * T::kFN + j, region, col[j]);
    wsc[j] = expert_scales(region, e);
  }

  f32x4 acc[T::kFM][T::kFN];
  // 16-row fragments of this wave with a live row (the rest are skipped)
  const int wave_rows = pend - p0 - wm * T::kWaveM;
  const int live_fm = wave_rows <= 0 ? 0 : (wave_rows >= T::kWaveM ? T::kFM : (wave_rows + 15) / 16);
  if constexpr (BLOCK) {
    // Activation scales of the block's rows: [128][KT] (zero for dead rows).
    for (int i = threadIdx.x; i < 128 * KT; i += blockDim.x) {
      const int rr = i / KT, kg = i % KT;
      const int pp = p0 + rr;
      sa_lds[i] = pp < pend ? ascales[static_cast<uint64_t>(src_row(pp)) * KT + kg] : 0.0f;
    }
    __syncthreads();
    BlockScaleFold fold{sa_lds, KT, wm, lane, {}};
    // The weight-scale rows are the same for every lane of the wave; with a
    // provably uniform address their per-k-tile reads are scalar loads,
    // counted apart from the vector-memory loads of the stage ring (a vector
    // load here would make the loop wait for every outstanding stage load).
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) fold.sw[j] = uniform_ptr(wsc[j] + (col[j] >> 7) * KT);
    w8a8v3::mainloop<T, BlockScaleFold, true>(plan, KT, smem, acc, fold, live_fm);
  } else {
    w8a8v3::mainloop<T, w8a8v3::NoFold, true>(plan, KT, smem, acc, w8a8v3::NoFold{}, live_fm);
  }

  const int r = lane & 15;
  // Per-channel form: every scale of this lane before the first store (the
  // stores share the workspace with the scale arrays, so a load between
  // stores would wait for them).
  float swv[T::kFN], sav[T::kFM][4];
  if constexpr (!BLOCK) {
#pragma unroll
    for (int j = 0; j < T::kFN; ++j) swv[j] = wsc[j][col[j] + r];
    // row scales in expert order: the token quantizer writes the token
    // scales to the h-scale array by position (stage 0), the hidden
    // quantizer its own (stage 1)
    const float *row_scales = at<float>(ws, L.hs);
#pragma unroll
    for (int i = 0; i < T::kFM; ++i)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int pp = p0 + w8a8v3::acc_row<T>(wm, i, lane, rr);
        sav[i][rr] = row_scales[pp < pend ? pp : p0];
      }
  }
#pragma unroll
  for (int i = 0; i < T::kFM; ++i) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int pp = p0 + w8a8v3::acc_row<T>(wm, i, lane, rr);
      if (pp >= pend) continue;
      if (STAGE == 0) {
        uint16_t *hrow = at<uint16_t>(ws, L.h) + static_cast<uint64_t>(pp) * N;
#pragma unroll
        for (int j = 0; j < T::kFN / 2; ++j) {
          const int c = col[j] + r;
          const float gv = BLOCK ? acc[i][j][rr] : acc[i][j][rr] * sav[i][rr] * swv[j];
          const float uv = BLOCK ? acc[i][j + T::kFN / 2][rr]
                                 : acc[i][j + T::kFN / 2][rr] * sav[i][rr] * swv[j + T::kFN / 2];
          hrow[c] = static_cast<uint16_t>(f32_to_bf16(silu_mul(gv, uv)));
        }
      } else {
        uint16_t *yrow = at<uint16_t>(ws, L.y) + static_cast<uint64_t>(pp) * N;
#pragma unroll
        for (int j = 0; j < T::kFN; ++j) {
          const int c = col[j] + r;
          yrow[c] = static_cast<uint16_t>(
              f32_to_bf16(BLOCK ? acc[i][j][rr] : acc[i][j][rr] * sav[i][rr] * swv[j]));
        }
      }
    }
  }
}

// Grouped GEMM on 256 x 256 tiles (the half-step main loop of w8a8_v4.h,
// 8 waves, one block per CU) for the per-channel form. A weight strip (256
// columns x K) is streamed once per 256 routed rows of its expert instead of
// once per 128: with 128-row tiles, the tiles sharing a strip drift apart
// and miss in L2 (measured: the Mixtral gate/up GEMM fetched twice its
// weight bytes from HBM). Row tiles are the 256-row tiles of all experts
// (the second prefix the sort writes); the 1-D tile order is column-major as
// above. STAGE 0: 128 h-columns per block (each wave column's fragments are
// its gate tiles, then the up tiles of the same columns); STAGE 1: 256
// columns per block.
using GemmTile256 = w8a8v4::Tile<256, 256, 4, 4, 2>;

// Block scales (128 x 128 weight blocks, per-token-per-128-column activation
// scales) on the 256 x 256 tile, whose accumulators leave no registers for a
// fresh set per k-tile: the accumulators hold acc' = (sum so far) / sigma_kt
// with sigma_kt = a_kt(row) w_kt(column block), so before k-tile kt's MFMAs
// add its products they are multiplied by sigma_{kt-1} / sigma_kt, and the
// epilogue multiplies by the last sigma. A zero scale only belongs to an
// all-zero group, whose products are zero, so each scale sequence carries the
// last nonzero value forward (any nonzero sigma is then exact) and starts
// at 1. The row ratios a_{kt-1} / a_kt live in LDS [KT][256]; a wave's
// column block ratios (gate and up for gate/up, one block for down) in LDS.
constexpr int kT256MaxKT = 24;  // LDS: 24 KiB of row ratios beside the 128 KiB ring

template <int STAGE>
struct BlockRescale256 {
  using T = GemmTile256;
  static_assert(T::kFN >= T::kFM, "apply(o) rescales column fragment o");
  typedef const __attribute__((address_space(3))) float *lds_ptr;
  lds_ptr ra;       // [KT][256]: row ratios
  lds_ptr rw;       // this wave: [kT256MaxKT] gate (or down) block ratios, then (STAGE 0) up
  int row0;         // the lane's row of fragment 0 in the tile (swapped layout: one row per
                    // lane and fragment)
  float m[T::kFM];  // this k-tile's multipliers of the lane's rows
  int kt = 0;
  LF_DEVICE void load(int part) {
    const float wk = rw[part * kT256MaxKT + kt];
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) m[i] = ra[kt * 256 + row0 + 32 * i] * wk;
  }
  LF_DEVICE void begin(int k) {
    kt = k;
    load(0);
  }
  template <class A>
  LF_DEVICE void apply(int o, A &acc) {
    // the up fragments (o is a compile-time unrolled index: no runtime branch)
    if constexpr (STAGE == 0) {
      if (o == T::kFN / 2) load(1);
    }
#pragma unroll
    for (int i = 0; i < T::kFM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][o][r] *= m[i];
  }
};


// QUANT (block-scaled gate/up only): the epilogue also quantizes h, writing
// the hidden quantizer's e4m3 codes and per-128-column scales instead of
// bf16 h (see the STAGE 0 epilogue below).
// bid: the block's index in the GEMM's part of the grid (blockIdx.x when the
// GEMM is the whole grid). gate(tile, rows) runs once the tile's expert and
// rows are known and before any of its activation rows or row scales is
// read; false: the tile is not computed (AnyTile: every tile runs). A gated
// tile reads its row scales with agent-scope loads: they were written in
// the same launch, and a tile's first and last scales share 128-byte lines
// with its neighbours', which a block of the same XCD may have read earlier.
struct AnyTile {
  LF_DEVICE bool operator()(int, int) const { return true; }
};
template <int STAGE, bool BLOCK = false, bool QUANT = false, class Gate = AnyTile>
__device__ __forceinline__ void grouped_gemm_t256(const int32_t *counts, const MoeDesc &d, const uint8_t *w0,
                                  const uint8_t *w1, uint8_t *ws, int bid = -1,
                                  const Gate &gate = Gate{}) {
  constexpr bool kGated = !std::is_same<Gate, AnyTile>::value;
  static_assert(!QUANT || (STAGE == 0 && BLOCK), "the fused quantizer is the block-scaled gate/up's");
  using T = GemmTile256;
  constexpr int BM = T::kBM;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[T::kSmem];
  __shared__ __attribute__((aligned(16))) float ra_lds[BLOCK ? kT256MaxKT * BM : 1];
  __shared__ float rw_lds[BLOCK ? T::kWgn * 2 * kT256MaxKT : 1];
  __shared__ float sw_last[BLOCK ? T::kWgn * 2 : 1];

  const int Tn = live_rows(counts, 1 << 30);
  if (Tn == 0) return;
  const MoeLayout L(d, Tn);
  const int E = d.experts;
  const int32_t *tiles = at<int32_t>(ws, L.tiles) + (E + 1);
  const WeightHeader &h0 = header_of(w0);
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int N = static_cast<int>(h0.rows);
  // the 32-bit activation offsets of the load plan (the launch geometry
  // picks this form only when they fit)
  const uint64_t a_rows = STAGE == 0 ? static_cast<uint64_t>(Tn) : static_cast<uint64_t>(Tn) * d.top_k;
  if (a_rows * static_cast<uint64_t>(K) >= (uint64_t(1) << 32)) return;
  const int gx = STAGE == 0 ? N / (T::kBN / 2) : N / T::kBN;
  int bx, by;
  if (!w8a8v3::tile_of_block(bid < 0 ? static_cast<int>(blockIdx.x) : bid, gx, tiles[E], tiles[E], bx,
                             by)) {
    return;
  }
  const TileExpert te = find_tile_expert(tiles, at<int32_t>(ws, L.offsets), E, by);
  const int e = te.e;
  const int p0 = te.row_begin + (by - te.first_tile) * BM;
  const int pend = te.row_end;
  // (the tile's live rows: pend is the end of its expert's rows)
  if (!gate(by, pend - p0 < BM ? pend - p0 : BM)) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / T::kWgn, wn = wave % T::kWgn;
  const int32_t *sorted = at<int32_t>(ws, L.sorted);
  auto src_row = [&](int p) { return STAGE == 0 ? sorted[p] / d.top_k : p; };

  auto slot = [&](int s, const uint8_t *&region, int &t, int &ocol) {
    if (STAGE == 0) {
      const int sw = s / (2 * T::kFN), f = s % (2 * T::kFN);
      const bool up = f >= T::kFN;
      ocol = bx * (T::kBN / 2) + sw * (T::kWaveN / 2) + 16 * (up ? f - T::kFN : f);
      region = up ? w1 : w0;
    } else {
      ocol = bx * T::kBN + 16 * s;
      region = w0;
    }
    t = ocol >> 4;
  };

  const uint8_t *abase = at<uint8_t>(ws, STAGE == 0 ? L.xq : L.hq);
  // Row scales of the tile in expert order (both stages find them in the
  // h-scale array: the token quantizer writes the token scales there by
  // position, the hidden quantizer later its own), one per thread of the
  // first 256, loaded before the main loop and parked in LDS after it.
  __shared__ float sa_tile[BM];
  float sa_mine = 0.0f;
  if constexpr (!BLOCK) {
    const float *row_scales = at<float>(ws, L.hs);
    if (threadIdx.x < BM) {
      const int i = p0 + static_cast<int>(threadIdx.x) < pend ? p0 + threadIdx.x : p0;
      if constexpr (kGated) {
        sa_mine = __hip_atomic_load(row_scales + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        sa_mine = row_scales[i];
      }
    }
  } else {
    // Ratio tables (see BlockRescale256): threads 0..255 one tile row each
    // (its activation scales in token order for gate/up, expert order for
    // down; sa_mine <- the last nonzero one), threads 256.. one (wave
    // column, weight block) each.
    if (KT > kT256MaxKT) return;  // the launch geometry never selects this form then
    const float *ascales = at<float>(ws, STAGE == 0 ? L.xs : L.hs);
    const int tid = threadIdx.x;
    // Each thread issues all of its scale loads before the first use (one
    // memory latency instead of one per k-tile).
    float sv[kT256MaxKT];
    if (tid < BM) {
      const int pp = p0 + tid;
      const bool live = pp < pend;
      const float *sr = ascales + static_cast<uint64_t>(src_row(live ? pp : p0)) * KT;
#pragma unroll
      for (int kt = 0; kt < kT256MaxKT; ++kt) sv[kt] = kt < KT ? sr[kt] : 0.0f;
      float prev = 1.0f;
#pragma unroll
      for (int kt = 0; kt < kT256MaxKT; ++kt) {
        if (kt < KT) {
          const float r = live ? carry_ratio(sv[kt], prev) : 1.0f;
          ra_lds[kt * BM + tid] = kt == 0 ? 1.0f : r;
        }
      }
      sa_mine = prev;
    } else if (tid < BM + 2 * T::kWgn) {
      const int cw = (tid - BM) >> 1, part = (tid - BM) & 1;
      const uint8_t *region = STAGE == 0 && part ? w1 : w0;
      const int nb = STAGE == 0 ? (bx * (T::kBN / 2) + cw * (T::kWaveN / 2)) >> 7
                                : (bx * T::kBN + cw * T::kWaveN) >> 7;
      const float *sw = expert_scales(region, e) + static_cast<uint64_t>(nb) * KT;
#pragma unroll
      for (int kt = 0; kt < kT256MaxKT; ++kt) sv[kt] = kt < KT ? sw[kt] : 0.0f;
      float prev = 1.0f;
#pragma unroll
      for (int kt = 0; kt < kT256MaxKT; ++kt) {
        if (kt < KT) {
          const float r = carry_ratio(sv[kt], prev);
          rw_lds[(2 * cw + part) * kT256MaxKT + kt] = kt == 0 ? 1.0f : r;
        }
      }
      sw_last[2 * cw + part] = prev;
    }
    __syncthreads();
  }
  // A offsets from the token (or assignment) array: rows x K < 2^32 (the
  // launch geometry picks this form only then).
  w8a8v4::Plan<T> plan;
  plan.a_base = w8a8v3::uniform_ptr(abase);
#pragma unroll
  for (int q = 0; q < T::kAIns; ++q) {
    const int tr = w8a8v4::a_load_row<T>(wave, q, lane);
    const int p = p0 + tr < pend ? p0 + tr : p0;  // dead rows re-read the first row
    plan.a_off[q] = static_cast<uint32_t>(src_row(p)) * static_cast<uint32_t>(K) +
                    w8a8v4::a_load_slot(tr, lane) * 32;
  }
#pragma unroll
  for (int q = 0; q < T::kBIns; ++q) {
    const uint8_t *region;
    int t, ocol;
    slot(w8a8v4::b_load_tile<T>(wave, q), region, t, ocol);
    plan.b_base[q] = w8a8v3::uniform_ptr(expert_tiles(region, e) + static_cast<uint64_t>(t) * KT * kTileBytes);
  }
  plan.b_lane = lane * 16;
  w8a8v4::f32x16 acc[T::kFM][T::kFN];
  // 32-row fragments of this wave with a live row (an expert's last tile is
  // usually partial, and small experts fill a few rows of one tile).
  const int live_rows_wave = pend - (p0 + wm * T::kWaveM);
  const int live_fm = live_rows_wave <= 0 ? 0 : live_rows_wave >= T::kWaveM ? T::kFM
                                                                           : (live_rows_wave + 31) / 32;
  // A wave whose 32 A rows are all past the tile's last row issues no A
  // loads (a tile of a small expert then moves its weights and little
  // else through the load path).
  const bool a_loads = p0 + 16 * T::kAIns * wave < pend;
  // Per-channel column scales of the block, one per thread of the first 256
  // (STAGE 1: its 256 output columns; STAGE 0: its 128 gate, then 128 up
  // columns), loaded before the main loop and parked in LDS after it.
  float sw_mine = 0.0f;
  if constexpr (!BLOCK) {
    const int n = static_cast<int>(threadIdx.x);
    if (n < T::kBN) {
      sw_mine = STAGE == 0 ? expert_scales(n < T::kBN / 2 ? w0 : w1, e)[bx * (T::kBN / 2) + (n & (T::kBN / 2 - 1))]
                           : expert_scales(w0, e)[bx * T::kBN + n];
    }
  }
  // The MFMAs run with swapped operands (mainloop SWAP): lane l holds tile
  // row wm * 64 + 32 i + l % 32 of fragment i and, for element 4 g + q of
  // fragment j, wave-tile column 32 j + 8 g + 4 (l / 32) + q. One row scale
  // (and block-scale multiplier) per lane and fragment instead of 16 keeps
  // registers free for the loop, and the epilogue stages 4 columns (8 bytes)
  // per LDS write.
  if constexpr (BLOCK) {
    typedef const __attribute__((address_space(3))) float *lds_ptr;
    BlockRescale256<STAGE> rs{(lds_ptr)(ra_lds), (lds_ptr)(rw_lds + 2 * wn * kT256MaxKT),
                              wm * T::kWaveM + (lane & 31), {}, 0};
    w8a8v4::mainloop<T, true, BlockRescale256<STAGE>, true>(plan, KT, smem, acc, live_fm, rs, a_loads);
  } else {
    w8a8v4::mainloop<T, true, w8a8v4::NoRescale, true>(plan, KT, smem, acc, live_fm,
                                                        w8a8v4::NoRescale{}, a_loads);
  }

  __shared__ float sw_tile[BLOCK ? 1 : T::kBN];
  if (threadIdx.x < BM) sa_tile[threadIdx.x] = sa_mine;
  if constexpr (!BLOCK) {
    if (threadIdx.x < T::kBN) sw_tile[threadIdx.x] = sw_mine;
  }
  // Column scale of wave-tile column cc of part `part` (0: gate or down
  // columns, 1: up columns).
  auto col_scale = [&](int part, int cc) -> float {
    if constexpr (BLOCK) {
      return sw_last[2 * wn + part];
    } else {
      return STAGE == 0 ? sw_tile[part * (T::kBN / 2) + wn * (T::kWaveN / 2) + cc]
                        : sw_tile[wn * T::kWaveN + cc];
    }
  };
  const int rl = lane & 31, c4 = 4 * (lane >> 5);
  // The output goes through LDS in 16-byte row chunks (w8a8v4::StageTile):
  // STAGE 0 stages 32 rows x 64 h-columns of bf16 per pass, STAGE 1 32 rows
  // x 128 columns of bf16; each lane writes 4 consecutive columns at a time.
  w8a8v4::epilogue_barrier();
  const int pw = p0 + wm * T::kWaveM;
  if constexpr (QUANT) {
    // SwiGLU -> bf16 (the value the unfused path stores as h) -> the hidden
    // quantizer. The block's 128 h-columns are one scale group (bx): the
    // whole 256 x 128 bf16 tile is staged in LDS, then each wave quantizes
    // 32 of its rows as lf_moe_quant_hidden does (16 lanes per row, 8
    // values each: amax over the 16 lanes, ratio = 448 / amax, codes =
    // e4m3_rne_sat(h * ratio), scale amax / 448; a zero group gets zero codes
    // and scale 0), so codes and scales are bit for bit that kernel's.
    constexpr int kPitch = T::kBN / 2 + 8;  // staged bf16 per row: 128 + pad
    static_assert(T::kBN / 2 == 128, "a block's h-columns are one 128-column group");
    static_assert(BM * kPitch * 2 <= T::kSmem, "the h tile fits the stage ring");
    uint16_t *tile = reinterpret_cast<uint16_t *>(smem);
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
      const int row = wm * T::kWaveM + w8a8v4::acc_row_t<T>(i, lane);
      const float sa = sa_tile[row];
#pragma unroll
      for (int j = 0; j < T::kFN / 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int cc = 32 * j + 8 * g + c4;
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = acc[i][j][4 * g + q] * sa * col_scale(0, cc + q);
            const float uv = acc[i][j + T::kFN / 2][4 * g + q] * sa * col_scale(1, cc + q);
            b[q] = f32_to_bf16(silu_mul(gv, uv));
          }
          *reinterpret_cast<uint2 *>(tile + row * kPitch + wn * (T::kWaveN / 2) + cc) =
              uint2{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
        }
    }
    __syncthreads();
    uint8_t *hq = at<uint8_t>(ws, L.hq);
    float *hs = at<float>(ws, L.hs);
    const int groups = N >> 7, hcol0 = bx * (T::kBN / 2);
    const int ch = lane & 15;
    constexpr int kRowsPerWave = BM / T::kWaves;
#pragma unroll
    for (int it = 0; it < kRowsPerWave / 4; ++it) {
      const int row = wave * kRowsPerWave + 4 * it + (lane >> 4);
      const uint4 v = *reinterpret_cast<const uint4 *>(tile + row * kPitch + ch * 8);
      float amax = bf16x8_amax(v, 0.0f);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
      const bool zero = amax == 0.0f;
      const float ratio = zero ? 0.0f : 448.0f / amax;
      const int p = p0 + row;
      if (p < pend) {
        *reinterpret_cast<uint2 *>(hq + static_cast<uint64_t>(p) * N + hcol0 + ch * 8) =
            bf16x8_encode(v, ratio, zero);
        if (ch == 0) hs[static_cast<uint64_t>(p) * groups + bx] = zero ? 0.0f : amax / 448.0f;
      }
    }
  } else if constexpr (STAGE == 0) {
    using Stage = w8a8v4::StageTile<uint16_t, 32, T::kWaveN / 2>;
    static_assert(Stage::kBytes * T::kWaves <= T::kSmem, "staging fits the stage ring");
    const Stage st{reinterpret_cast<uint16_t *>(smem + wave * Stage::kBytes)};
    uint16_t *h = at<uint16_t>(ws, L.h);
    const int col0 = bx * (T::kBN / 2) + wn * (T::kWaveN / 2);
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
      const float sa = sa_tile[wm * T::kWaveM + w8a8v4::acc_row_t<T>(i, lane)];
#pragma unroll
      for (int j = 0; j < T::kFN / 2; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int cc = 32 * j + 8 * g + c4;
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = acc[i][j][4 * g + q] * sa * col_scale(0, cc + q);
            const float uv = acc[i][j + T::kFN / 2][4 * g + q] * sa * col_scale(1, cc + q);
            b[q] = f32_to_bf16(silu_mul(gv, uv));
          }
          st.put4(rl, cc, b);
        }
      const int p_i = pw + 32 * i;
      st.flush(lane, [&](int row) -> uint16_t * {
        return p_i + row < pend ? h + static_cast<uint64_t>(p_i + row) * N + col0 : nullptr;
      });
    }
  } else {
    using Stage = w8a8v4::StageTile<uint16_t, 32, T::kWaveN>;
    static_assert(Stage::kBytes * T::kWaves <= T::kSmem, "staging fits the stage ring");
    const Stage st{reinterpret_cast<uint16_t *>(smem + wave * Stage::kBytes)};
    uint16_t *y = at<uint16_t>(ws, L.y);
    const int col0 = bx * T::kBN + wn * T::kWaveN;
#pragma unroll
    for (int i = 0; i < T::kFM; ++i) {
      const float sa = sa_tile[wm * T::kWaveM + w8a8v4::acc_row_t<T>(i, lane)];
#pragma unroll
      for (int j = 0; j < T::kFN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int cc = 32 * j + 8 * g + c4;
          uint32_t b[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) b[q] = f32_to_bf16(acc[i][j][4 * g + q] * sa * col_scale(0, cc + q));
          st.put4(rl, cc, b);
        }
      const int p_i = pw + 32 * i;
      st.flush(lane, [&](int row) -> uint16_t * {
        return p_i + row < pend ? y + static_cast<uint64_t>(p_i + row) * N + col0 : nullptr;
      });
    }
  }
}

// Per-channel profiles on the 256-row tiles (e.g. Mixtral): the hidden
// quantizer as the first counted step of the down launch
// (lf_moe_down_t256_aq), so the plan has no lf_moe_quant_hidden launch. Per-
// token scales need a whole row of h (I columns from every gate/up column
// block), so the quantizer cannot live in the gate/up epilogue; here
// kQuantBlocks blocks at the head of the grid quantize h in chunks of
// kChunkRows rows (one wave per row: the standalone quantizer's code, its
// stores written through, phases.h; rows of 8193-16384 columns by wave
// pairs, two rows a pair) and count each row into the counter of
// its 256-row tile; a down tile starts its loads once its tile's counter
// holds the tile's row count. The counters live in the operation's sync
// area (the fifth operand, at a fixed offset of the workspace: error word,
// done counter, one 128-byte line per row tile), left at zero by the last
// down block of every launch.
// RB rows of h held by S waves in registers (S = 2 for rows of 8193-16384
// columns, e.g. Mixtral's I = 14336, that the one-wave forms hold only with
// 32 chunks per lane, past this kernel's register budget): wave part q of
// the rows holds 16-byte chunks [q per, (q + 1) per) of each of its RB rows
// as the one-wave form holds a whole row (C chunks per lane and row, every
// load of the RB rows in flight at once), a row's amax is the max of the S
// waves' maxima (through red, RB floats per wave in LDS), then each wave
// encodes its own chunks. A max is exact in any order, so amax, ratio,
// codes and scale are those of the one-wave forms. Rows p0 .. p0 + RB - 1;
// those at or past A load and store nothing. Every wave of the block calls
// it (it holds a block barrier).
template <int C, int S, int RB>
LF_DEVICE void quantize_rows_split(const uint16_t *h, int I, int p0, int A, uint8_t *hq, float *hs,
                                   float *red, int wave) {
  const int lane = threadIdx.x & 63, part = wave % S;
  const int chunks = I >> 3, per = (chunks + S - 1) / S;
  const int c0 = part * per, c1 = c0 + per < chunks ? c0 + per : chunks;
  u32x4 v[RB][C];
  static_for<RB>([&](auto b) {
    const bool live = p0 + b < A;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(h + static_cast<uint64_t>(live ? p0 + b : 0) * I);
    static_for<C>([&](auto c) {
      const int idx = c0 + lane + 64 * c;
      v[b][c] = (live && idx < c1) ? src[idx] : u32x4{0u, 0u, 0u, 0u};
    });
  });
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
    if (lane == 0) red[RB * wave + b] = amax;
  });
  __syncthreads();
  static_for<RB>([&](auto b) {
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < S; ++q) amax = fmaxf(amax, red[RB * (wave - part + q) + b]);
    const bool live = p0 + b < A, zero = amax == 0.0f;
    const float ratio = zero ? 0.0f : 448.0f / amax;
    static_for<C>([&](auto c) { opaque(v[b][c]); });
    uint8_t *dst = hq + static_cast<uint64_t>(live ? p0 + b : 0) * I;
    static_for<C>([&](auto c) {
      const int idx = c0 + lane + 64 * c;
      const uint32_t lo = e4m3x4_from_bf16(v[b][c][0], v[b][c][1], ratio);
      const uint32_t hi = e4m3x4_from_bf16(v[b][c][2], v[b][c][3], ratio);
      if (live && idx < c1) store_codes8<true>(dst + 8 * idx, zero ? 0u : lo, zero ? 0u : hi);
    });
    if (live && part == 0 && lane == 0) store_scale<true>(hs + p0 + b, zero ? 0.0f : amax / 448.0f);
  });
}

LF_DEVICE void moe_down_aq(const int32_t *counts, const MoeDesc &d, const uint8_t *wd, uint8_t *ws,
                           uint8_t *sync_area) {
  __shared__ phase::Flag flag;
  __shared__ int32_t tab[2 * 257];  // row offsets [E + 1], then the 256-row tile prefix [E + 1]
  constexpr int kHeldRows = 64;
  __shared__ int row_tile[kHeldRows];  // the 256-row tile of each held row (-1: none)
  __shared__ float red[2 * kChunkRows];  // per-wave row maxima (quantize_rows_split)
  const int Tn = live_rows(counts, 1 << 30);
  if (Tn == 0) return;
  const MoeLayout L(d, Tn);
  const int E = d.experts, A = Tn * d.top_k, I = d.inter;
  const int32_t *offsets = at<int32_t>(ws, L.offsets);
  const int32_t *tiles = at<int32_t>(ws, L.tiles) + (E + 1);
  const int b = static_cast<int>(blockIdx.x);
  if (b < kQuantBlocks) {
    const phase::Sync sync{reinterpret_cast<int *>(sync_area), 1};
    for (int i = threadIdx.x; i <= E; i += blockDim.x) {
      tab[i] = offsets[i];
      tab[E + 1 + i] = tiles[i];
    }
    __syncthreads();
    const uint16_t *h = at<uint16_t>(ws, L.h);
    uint8_t *hq = at<uint8_t>(ws, L.hq);
    float *hs = at<float>(ws, L.hs);
    const int wave = static_cast<int>(threadIdx.x) >> 6, lane = threadIdx.x & 63;
    // waves per row (block-uniform): rows of 8193-16384 columns by wave
    // pairs, each wave holding halves of two rows (up to 14336 columns: 14
    // chunks per lane and row) or of one (16 chunks); one wave per row else
    const int S = I > 8192 && I <= 16384 ? 2 : 1;
    const int RB = S == 2 && I <= 14336 ? 2 : 1;
    const int R = kChunkRows / S * RB;  // rows per chunk
    const int first = wave / S * RB;    // this wave's first row in the chunk
    const int chunks = (A + R - 1) / R;
    int held = 0;  // rows quantized and not yet counted (block-uniform)
    for (int c = b; c < chunks; c += kQuantBlocks) {
      const int p0 = c * R + first;
      if (RB == 2) {
        quantize_rows_split<14, 2, 2>(h, I, p0, A, hq, hs, red, wave);
      } else if (S == 2) {
        quantize_rows_split<16, 2, 1>(h, I, p0, A, hq, hs, red, wave);
      } else if (p0 < A) {
        const uint64_t off = static_cast<uint64_t>(p0) * I;
        // (the two-pass form above 16384 columns)
        quantize_row_wave<true, 16>(h + off, I, hq + off, hs + p0);
      }
      if (lane == 0 && wave % S == 0) {
        for (int r = 0; r < RB; ++r) {
          const int p = p0 + r;
          int tile = -1;
          if (p < A) {
            // the expert of row p: offsets[e] <= p < offsets[e + 1]
            int lo = 0, hi = E;
            while (hi - lo > 1) {
              const int mid = (lo + hi) >> 1;
              if (tab[mid] <= p) {
                lo = mid;
              } else {
                hi = mid;
              }
            }
            tile = tab[E + 1 + lo] + ((p - tab[lo]) >> 8);
          }
          row_tile[held + first + r] = tile;
        }
      }
      held += R;
      // The rows are counted once the block's stores of them have completed,
      // when the list is full or after the block's last chunk: a down tile
      // cannot take this CU before this block ends (one block per CU), so
      // counting chunk by chunk would only put a store wait between chunks.
      if (held + R > kHeldRows || c + kQuantBlocks >= chunks) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) {
          // runs of rows of one tile as one add
          for (int w = 0; w < held;) {
            int n = 1;
            while (w + n < held && row_tile[w + n] == row_tile[w]) ++n;
            if (row_tile[w] >= 0) {
              __hip_atomic_fetch_add(sync.band(0, row_tile[w]), n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            w += n;
          }
        }
        __syncthreads();  // row_tile is rewritten from the start
        held = 0;
      }
    }
    return;
  }
  const phase::Sync sync{reinterpret_cast<int *>(sync_area), tiles[E]};
  const auto gate = [&](int tile, int rows) {
    return phase::wait_for(sync, sync.band(0, tile), rows, flag);
  };
  grouped_gemm_t256<1, false, false>(counts, d, wd, wd, ws, b - kQuantBlocks, gate);
  phase::finish(sync, static_cast<int>(gridDim.x) - kQuantBlocks, 1, flag);
}

// --- grouped GEMV form ------------------------------------------------------------
// Profiles of at most 32 tokens: every expert holds at most 32 rows (a token
// picks an expert once), and the GEMMs are bound by streaming the touched
// experts' weights, not by the matrix pipes. Work items are (expert with
// rows, group of kGemvWaves consecutive 16-column tiles), from the sort's
// list of experts with rows; a fixed grid of blocks loops over them (no
// blocks for empty experts, whose dispatch slots would delay live ones). A
// wave takes one tile of the item (for gate/up the gate and the up tile of
// the same 16 h-columns) and streams it over all of K, kGemvRing k-tiles
// ahead, against the expert's rows in 16-row chunks (an expert of more than
// 16 rows re-reads its tiles from L2 for each further chunk), with
// v_mfma_scale_f32_16x16x128_f8f6f4: a 128-deep k-tile is one MFMA and one
// scale block, and a packed weight tile is its B operand as stored (lane l:
// column l % 16, k = 32 (l / 16) + 0..31 from the two 1 KiB halves). Lane l
// holds A row l % 16 of the chunk at the same k bytes, gathered through the
// sorted ids for gate/up. Block scales: each k-tile's product is folded with
// s_a[row][kt] (a per-wave LDS table, so no block barrier) and s_w[column
// block][kt] (scalar loads); per-channel scales multiply the sums in the
// epilogue. The weight loads of an item are issued first, the dependent
// chain its activation rows need (offsets, sorted ids, scales) after them.
constexpr int kGemvWaves = 4;
constexpr int kGemvRing = 4;
constexpr int kGemvRows = 16;

// 16 bytes at base + off through a global-address-space pointer: a
// global_load (vector-memory counter only) rather than a flat load, which
// the compiler must also count as a possible LDS access and wait for as one.
LF_DEVICE u32x4 gload16(const uint8_t *base, uint32_t off) {
  typedef const __attribute__((address_space(1))) uint8_t gbyte;
  typedef const __attribute__((address_space(1))) u32x4 gvec;
  return *reinterpret_cast<gvec *>((gbyte *)base + off);
}

template <int STAGE, bool BLOCK>
LF_DEVICE void grouped_gemv(const int32_t *counts, const MoeDesc &d, const uint8_t *w0,
                            const uint8_t *w1, uint8_t *ws) {
  constexpr int NW = STAGE == 0 ? 2 : 1;
  constexpr int D = kGemvRing;
  // Block form: each wave's activation scales of its row chunk, [KT][16],
  // KT <= 32 (the host rejects larger K for 128-column groups).
  __shared__ __attribute__((aligned(16))) float sa_lds[BLOCK ? kGemvWaves * kGemvRows * 32 : 4];
  const int Tn = live_rows(counts, 1 << 30);
  if (Tn == 0) return;
  const MoeLayout L(d, Tn);
  const WeightHeader &h0 = header_of(w0);
  const int K = static_cast<int>(h0.columns);
  const int KT = K >> 7;
  const int N = static_cast<int>(h0.rows);
  if (BLOCK && KT > 32) return;
  // Shapes the form is laid out for (the launch geometry only picks it for
  // them): whole 4-tile column groups, and activation offsets that fit the
  // 32-bit per-lane offsets of the loads.
  const uint64_t a_rows = STAGE == 0 ? static_cast<uint64_t>(Tn) : static_cast<uint64_t>(Tn) * d.top_k;
  if ((N & 63) != 0 || a_rows * static_cast<uint64_t>(K) >= (uint64_t(1) << 32)) return;
  if (blockDim.x != 64 * kGemvWaves) return;  // the item layout's block (the geometry's)
  const int E = d.experts;
  const int groups = (N >> 4) / kGemvWaves;
  const int32_t *live = at<int32_t>(ws, L.tiles) + 2 * E + 2;  // [0]: count, then ids
  const int nlive = live[0];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int32_t *offsets = at<int32_t>(ws, L.offsets);
  // Row chunks are items of their own: expert j of the live list has
  // ceil(rows_j / 16) chunks; items (j, chunk 0, group) come first, j-major,
  // then the further chunks, numbered by extra[j] = sum over i < j of
  // (chunks_i - 1): item nlive * groups + x * groups + group is chunk
  // 1 + x - extra[j] of the expert j with extra[j] <= x < extra[j + 1]. A
  // further chunk then streams its tiles in another block beside the first
  // chunk, not after it in the same block (with 17-32 rows that sequence set
  // the kernel's length). One thread per live expert (E <= 256 = blockDim.x)
  // and a wave scan build the prefix in LDS.
  __shared__ int extra[257];
  __shared__ int wave_extra[kGemvWaves];
  {
    const int t = static_cast<int>(threadIdx.x);
    int mine = 0;
    if (t < nlive) {
      const int ex = live[1 + t];
      mine = (offsets[ex + 1] - offsets[ex] + kGemvRows - 1) / kGemvRows - 1;
      mine = mine < 0 ? 0 : mine;
    }
    int incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int v = __shfl_up(incl, off);
      if (lane >= off) incl += v;
    }
    if (lane == 63) wave_extra[wave] = incl;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wave_extra[w];
    extra[t + 1] = before + incl;
    if (t == 0) extra[0] = 0;
    __syncthreads();
  }
  const int first_items = nlive * groups;
  const int items = (nlive + extra[nlive]) * groups;
  const int32_t *sorted = at<int32_t>(ws, L.sorted);
  auto src_row = [&](int p) { return STAGE == 0 ? sorted[p] / d.top_k : p; };
  const uint8_t *abase = uniform_ptr(at<uint8_t>(ws, STAGE == 0 ? L.xq : L.hq));
  const float *ascales = at<float>(ws, STAGE == 0 ? L.xs : L.hs);
  float *sa_wave = sa_lds + (BLOCK ? wave * kGemvRows * 32 : 0);

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    int j = item / groups, chunk = 0;
    if (item >= first_items) {
      const int x = (item - first_items) / groups;
      int lo = 0, hi = nlive;  // extra[lo] <= x < extra[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (extra[mid] <= x) lo = mid; else hi = mid;
      }
      j = lo;
      chunk = 1 + x - extra[lo];
    }
    const int e = live[1 + j];
    const int nt = (item % groups) * kGemvWaves + wave;
    const int col = nt * 16 + (lane & 15);
    const uint8_t *region[NW];
    region[0] = w0;
    if constexpr (NW == 2) region[1] = w1;
    // Uniform bases (scalar registers) with 32-bit per-lane offsets: the
    // loads take the base + offset form instead of a 64-bit address each.
    const uint8_t *strip[NW];
    const float *wsc[NW], *wsc_blk[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      strip[i] = uniform_ptr(expert_tiles(region[i], e) + static_cast<uint64_t>(nt) * KT * kTileBytes);
      wsc[i] = expert_scales(region[i], e);
      // block form: the [KT] scales of this tile's 128-column block
      wsc_blk[i] = uniform_ptr(wsc[i] + (BLOCK ? (nt >> 3) * KT : 0));
    }
    u32x4 bw[D][NW][2];
    auto load_b = [&](int slot, int kt) {
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const uint32_t o = static_cast<uint32_t>(kt) * kTileBytes + lane * 16;
        bw[slot][i][0] = gload16(strip[i], o);
        bw[slot][i][1] = gload16(strip[i], o + 1024);
      }
    };
    const int pend = offsets[e + 1];
    const int c0 = offsets[e] + kGemvRows * chunk;
    if (c0 < pend) {
      const int rows = pend - c0 < kGemvRows ? pend - c0 : kGemvRows;
      // the weight ring's first D k-tiles, then the activation chain
      static_for<D>([&](auto j) { load_b(j, j < KT ? static_cast<int>(j) : KT - 1); });
      __builtin_amdgcn_sched_barrier(0);
      const int my_src = src_row(c0 + (r < rows ? r : 0));  // the source row of lane row r
      const uint32_t aoff = static_cast<uint32_t>(my_src) * static_cast<uint32_t>(K) + 32 * g;
      if constexpr (BLOCK) {
        // This wave's table, [KT][16] (k-major, so a lane's 4 rows of one
        // k-tile are one 16-byte read), zero for dead rows; the wave alone
        // reads it, in order after its writes. Lane l fills row l % 16 at
        // k-tiles l / 16 + 4 m: all its loads are issued together.
        constexpr int kMaxPer = 8;  // KT <= 32
        float v[kMaxPer];
        const float *srow = ascales + static_cast<uint64_t>(my_src) * KT;
        static_for<kMaxPer>([&](auto m) {
          const int kg = g + 4 * m;
          v[m] = srow[kg < KT ? kg : 0];
        });
        static_for<kMaxPer>([&](auto m) {
          const int kg = g + 4 * m;
          if (kg < KT) sa_wave[kg * 16 + r] = r < rows ? v[m] : 0.0f;
        });
      }
      f32x4 acc[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) acc[w] = f32x4{0.f, 0.f, 0.f, 0.f};
      // The k loop is branch-free (a branch in it makes the compiler wait
      // for every outstanding load at each k-tile, which drains the ring).
      u32x4 av[D][2];
      auto load_a = [&](int slot, int kt) {
        const uint32_t o = aoff + kt * 128;
        av[slot][0] = gload16(abase, o);
        av[slot][1] = gload16(abase, o + 16);
      };
      static_for<D>([&](auto j) { load_a(j, j < KT ? static_cast<int>(j) : KT - 1); });
      // One k-tile of ring slot j: MFMA(s) on the slot, then its refill D
      // k-tiles ahead (clamped to the last k-tile, so the loads are issued
      // unconditionally and the compiler's vmcnt waits stay exact), in this
      // order: sched_barrier keeps the scheduler from moving the refills,
      // which would shorten the ring. A k-tile past K (the ring's tail in
      // the runtime loop) re-reads the last one and contributes nothing: a
      // select, not a branch.
      auto k_step = [&](auto jc, int kt) {
          constexpr int j = decltype(jc)::value;
          const bool kt_live = kt < KT;
          const int ktc = kt_live ? kt : KT - 1;
          float swk[NW];
          f32x4 sa4;
          if constexpr (BLOCK) {
#pragma unroll
            for (int w = 0; w < NW; ++w) {
              const float v = sload(wsc_blk[w], ktc);
              swk[w] = kt_live ? v : 0.0f;
            }
            sa4 = *reinterpret_cast<const f32x4 *>(sa_wave + ktc * 16 + 4 * g);
          }
          const i32x8 af = __builtin_bit_cast(
              i32x8, __builtin_shufflevector(av[j][0], av[j][1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const i32x8 bf = __builtin_bit_cast(
                i32x8, __builtin_shufflevector(bw[j][w][0], bw[j][w][1], 0, 1, 2, 3, 4, 5, 6, 7));
            if constexpr (BLOCK) {
              const f32x4 step = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                  af, bf, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[w][q] += step[q] * (sa4[q] * swk[w]);
            } else {
              const f32x4 next = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                  af, bf, acc[w], 0, 0, 0, 127, 0, 127);
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[w][q] = kt_live ? next[q] : acc[w][q];
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          const int nk = kt + D < KT ? kt + D : KT - 1;
          load_b(j, nk);
          load_a(j, nk);
          __builtin_amdgcn_sched_barrier(0);
      };
      // A runtime loop of D-step groups: the compiler waits for every
      // outstanding load at the top of each group. (Unrolled over a
      // compile-time K it keeps the ring full, but its register use grows
      // with K: 256 VGPRs and AGPRs with spills at K = 4096.)
      for (int k0 = 0; k0 < KT; k0 += D) {
        static_for<D>([&](auto jc) { k_step(jc, k0 + decltype(jc)::value); });
      }
      // epilogue: lane holds rows 4 g + q of column col
      float sw[NW];
      if constexpr (!BLOCK) {
#pragma unroll
        for (int w = 0; w < NW; ++w) sw[w] = wsc[w][col];
      }
      const float *row_scales = at<float>(ws, L.hs);  // per-token scales in expert order
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = 4 * g + q;
        if (rr >= rows) continue;
        const int p = c0 + rr;
        const float sa = BLOCK ? 1.0f : row_scales[p];
        if constexpr (STAGE == 0) {
          const float gv = BLOCK ? acc[0][q] : acc[0][q] * sa * sw[0];
          const float uv = BLOCK ? acc[1][q] : acc[1][q] * sa * sw[1];
          at<uint16_t>(ws, L.h)[static_cast<uint64_t>(p) * N + col] =
              static_cast<uint16_t>(f32_to_bf16(silu_mul(gv, uv)));
        } else {
          at<uint16_t>(ws, L.y)[static_cast<uint64_t>(p) * N + col] =
              static_cast<uint16_t>(f32_to_bf16(BLOCK ? acc[0][q] : acc[0][q] * sa * sw[0]));
        }
      }
    }
  }
}

// --- combine -------------------------------------------------------------------
LF_DEVICE void combine(const int32_t *counts, const MoeDesc &d, uint8_t *ws, uint16_t *out) {
  const int T = live_rows(counts, 1 << 30);
  const int t = blockIdx.x;
  if (t >= T) return;
  const MoeLayout L(d, T);
  const int H = d.hidden;
  const float *w = at<float>(ws, L.topk_w) + static_cast<uint64_t>(t) * d.top_k;
  const int32_t *pos = at<int32_t>(ws, L.pos) + static_cast<uint64_t>(t) * d.top_k;
  const uint16_t *y = at<uint16_t>(ws, L.y);
  // eight columns per thread (H % 128 == 0); the k rows' loads are all
  // issued before the sum, whose terms are added in slot order j
  constexpr int kMaxK = 16;  // desc_ok bounds top_k
  const int k = d.top_k;
  for (int c = 8 * threadIdx.x; c < H; c += 8 * blockDim.x) {
    u32x4 v[kMaxK];
    static_for<kMaxK>([&](auto j) {
      if (j < k) v[j] = *reinterpret_cast<const u32x4 *>(y + static_cast<uint64_t>(pos[j]) * H + c);
    });
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    static_for<kMaxK>([&](auto j) {
      // product and sum each rounded (no fused multiply-add), as the combine
      // is defined: the output is then bit-identical to that definition for
      // the same y and weights
#pragma clang fp contract(off)
      if (j < k) {
        const float wj = w[j];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t word = v[j][q >> 1];
          const float prod = wj * bf16_to_f32((q & 1) ? word >> 16 : word & 0xffffu);
          acc[q] = acc[q] + prod;
        }
      }
    });
    u32x4 packed;
#pragma unroll
    for (int q = 0; q < 4; ++q) packed[q] = f32_to_bf16(acc[2 * q]) | (f32_to_bf16(acc[2 * q + 1]) << 16);
    *reinterpret_cast<u32x4 *>(out + static_cast<uint64_t>(t) * H + c) = packed;
  }
}

// The descriptor by value: held in registers for the whole kernel. A
// reference into the descriptor buffer would be read again from memory after
// every fence and barrier (each a load latency in the routing and sort loops).
LF_DEVICE MoeDesc desc_of(const int32_t *desc) { return *reinterpret_cast<const MoeDesc *>(desc); }

}  // namespace

extern "C" {

// The route step's operands carry the tokens x for both of its kernels
// (lf_moe_route does not read them; lf_moe_route_sort quantizes them).
__global__ __launch_bounds__(256) void lf_moe_route(const int32_t *counts, const int32_t *desc,
                                                    const float *logits, const uint16_t *,
                                                    uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d)) return;
  route(counts, d, logits, ws);
}

__global__ __launch_bounds__(1024) void lf_moe_sort_count(const int32_t *counts,
                                                          const int32_t *desc, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d)) return;
  sort_count(counts, d, ws);
}

__global__ __launch_bounds__(1024) void lf_moe_sort(const int32_t *counts, const int32_t *desc,
                                                    uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d)) return;
  sort_assignments(counts, d, ws);
}

__global__ __launch_bounds__(1024) void lf_moe_route_sort(const int32_t *counts, const int32_t *desc,
                                                         const float *logits, const uint16_t *x,
                                                         uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || blockDim.x != kSortThreads) return;
  route_sort_block(counts, d, logits, x, ws);
}

__global__ __launch_bounds__(256) void lf_moe_quant_tokens(const int32_t *counts,
                                                           const int32_t *desc,
                                                           const uint16_t *x, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d)) return;
  const int T = live_rows(counts, 1 << 30);
  const MoeLayout L(d, T);
  if (d.group != 0) {
    quant_rows(x, d.hidden, d.group, at<uint8_t>(ws, L.xq), at<float>(ws, L.xs), T);
    return;
  }
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  const uint64_t off = static_cast<uint64_t>(row) * d.hidden;
  const float sc = quantize_row_wave(x + off, d.hidden, at<uint8_t>(ws, L.xq) + off,
                                     at<float>(ws, L.xs) + row);
  // The per-token scale also in expert order, at the position of each of
  // the token's k assignments (from the sort), for the gate/up epilogue. It
  // goes to the h-scale array, which the hidden quantizer only writes after
  // the gate/up GEMM has consumed it.
  const int lane = threadIdx.x & 63;
  if (lane < d.top_k) at<float>(ws, L.hs)[at<int32_t>(ws, L.pos)[row * d.top_k + lane]] = sc;
}

__global__ __launch_bounds__(256) void lf_moe_quant_hidden(const int32_t *counts,
                                                           const int32_t *desc, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d)) return;
  const int T = live_rows(counts, 1 << 30);
  const MoeLayout L(d, T);
  quant_rows(at<uint16_t>(ws, L.h), d.inter, d.group, at<uint8_t>(ws, L.hq), at<float>(ws, L.hs),
             T * d.top_k);
}

// Per-channel weight scales with per-token activation scales (group 0) ...
__global__ __launch_bounds__(256) void lf_moe_gate_up(const int32_t *counts, const int32_t *desc,
                                                      const uint8_t *wg, const uint8_t *wu,
                                                      uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 0 || header_of(wg).magic != kWeightMagic) return;
  grouped_gemm<0, false>(counts, d, wg, wu, ws);
}

__global__ __launch_bounds__(256) void lf_moe_down(const int32_t *counts, const int32_t *desc,
                                                   const uint8_t *wd, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 0 || header_of(wd).magic != kWeightMagic) return;
  grouped_gemm<1, false>(counts, d, wd, wd, ws);
}

// The same on 256 x 256 tiles (per-channel form, profiles with >= 256
// routed rows per expert on average).
__global__ __launch_bounds__(512) void lf_moe_gate_up_t256(const int32_t *counts,
                                                           const int32_t *desc,
                                                           const uint8_t *wg, const uint8_t *wu,
                                                           uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 0 || header_of(wg).magic != kWeightMagic) return;
  grouped_gemm_t256<0>(counts, d, wg, wu, ws);
}

// The per-channel down GEMM on 256-row tiles, with the hidden quantizer as
// the launch's first counted step (moe_down_aq): (counts, desc, wd, ws,
// sync), sync the operation's counter area (lunaflux_fp8_moe_sync_offset),
// zero-filled once when allocated.
__global__ __launch_bounds__(512) void lf_moe_down_t256_aq(const int32_t *counts,
                                                           const int32_t *desc, const uint8_t *wd,
                                                           uint8_t *ws, uint8_t *sync) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 0 || header_of(wd).magic != kWeightMagic) return;
  moe_down_aq(counts, d, wd, ws, sync);
}

// The same on 128 x 128 block scales (rescaled accumulators, see
// BlockRescale256); K <= 24 x 128 for both GEMMs.
__global__ __launch_bounds__(512) void lf_moe_gate_up_t256_b128(const int32_t *counts,
                                                                const int32_t *desc,
                                                                const uint8_t *wg,
                                                                const uint8_t *wu, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 128 || header_of(wg).magic != kWeightMagic) return;
  grouped_gemm_t256<0, true>(counts, d, wg, wu, ws);
}

// The same with the hidden quantizer fused into the epilogue: writes h's
// e4m3 codes and per-128-column scales (the arrays lf_moe_quant_hidden
// fills), not bf16 h; the plan then has no lf_moe_quant_hidden launch.
__global__ __launch_bounds__(512) void lf_moe_gate_up_t256_b128_q(const int32_t *counts,
                                                                  const int32_t *desc,
                                                                  const uint8_t *wg,
                                                                  const uint8_t *wu, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 128 || header_of(wg).magic != kWeightMagic) return;
  grouped_gemm_t256<0, true, true>(counts, d, wg, wu, ws);
}

__global__ __launch_bounds__(512) void lf_moe_down_t256_b128(const int32_t *counts,
                                                             const int32_t *desc,
                                                             const uint8_t *wd, uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 128 || header_of(wd).magic != kWeightMagic) return;
  grouped_gemm_t256<1, true>(counts, d, wd, wd, ws);
}

// Small profiles (at most 32 tokens): the grouped GEMV form, either scale
// mode (the descriptor's group).
__global__ __launch_bounds__(256) void lf_moe_gate_up_gemv(const int32_t *counts,
                                                           const int32_t *desc,
                                                           const uint8_t *wg, const uint8_t *wu,
                                                           uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || header_of(wg).magic != kWeightMagic) return;
  if (d.group == 0) grouped_gemv<0, false>(counts, d, wg, wu, ws);
  else grouped_gemv<0, true>(counts, d, wg, wu, ws);
}

__global__ __launch_bounds__(256) void lf_moe_down_gemv(const int32_t *counts,
                                                        const int32_t *desc, const uint8_t *wd,
                                                        uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || header_of(wd).magic != kWeightMagic) return;
  if (d.group == 0) grouped_gemv<1, false>(counts, d, wd, wd, ws);
  else grouped_gemv<1, true>(counts, d, wd, wd, ws);
}

// ... and 128 x 128 block weight scales with per-token-per-128-column
// activation scales (group 128).
__global__ __launch_bounds__(256) void lf_moe_gate_up_b128(const int32_t *counts,
                                                           const int32_t *desc,
                                                           const uint8_t *wg, const uint8_t *wu,
                                                           uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 128 || header_of(wg).magic != kWeightMagic) return;
  grouped_gemm<0, true>(counts, d, wg, wu, ws);
}

__global__ __launch_bounds__(256) void lf_moe_down_b128(const int32_t *counts,
                                                        const int32_t *desc, const uint8_t *wd,
                                                        uint8_t *ws) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d) || d.group != 128 || header_of(wd).magic != kWeightMagic) return;
  grouped_gemm<1, true>(counts, d, wd, wd, ws);
}

__global__ __launch_bounds__(256) void lf_moe_combine(const int32_t *counts, const int32_t *desc,
                                                      uint8_t *ws, uint16_t *out) {
  const MoeDesc d = desc_of(desc);
  if (!desc_ok(d)) return;
  combine(counts, d, ws, out);
}

}  // extern "C"
