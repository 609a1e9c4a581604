/*
 * lunaflux_fp8.h - the FP8 projection path behind LunaFlux's kernel
 * catalog: the weight-region format that model/device_materialize writes,
 * the host-side pre-swizzle, the launch geometry a manifest records, and the
 * gfx950 kernel entry points (symbols in lunaflux_fp8.hsaco) with their
 * operand lists.
 *
 * Operand convention (kernels/launch_contract/paged_admit.mbt:76-107): every
 * kernel parameter is a device region, in canonical order runtime inputs,
 * semantic inputs (activation first, then weights in TensorRef order),
 * outputs, workspace. No scalars cross (kernels/launch_contract/
 * operands.mbt:1-13): the live row count M is read on the device from the
 * StepCounts descriptor int32[5] = {prefill_rows, decode_rows, total_rows,
 * query_tokens, page_entries} (engine/device_step/stage.mbt:59-68), element
 * 3; N and K are read from the weight region header. The grid is sized for
 * the profile's max_query_tokens (kernels/launch_contract/
 * paged_profile.mbt:7-13) and blocks past the live M exit early.
 */
#ifndef LUNAFLUX_FP8_H
#define LUNAFLUX_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- weight region format ---------------------------------------------- */
/*
 * One weight TensorRef = one region (engine/execution_manifest_file/
 * derive.mbt:163-173), laid out as
 *   [256-byte header | E x tile block | E x scale block]
 * Tile block of one expert: the [N, K] e4m3 matrix cut into 16 x 128 tiles,
 * tile (nt, kt) at ((nt * K/128) + kt) * 2048. Inside a tile the bytes are in
 * MFMA fragment order: half h (0, 1) holds 64 lanes x 16 bytes, and lane l's
 * 16 bytes at h*1024 + l*16 are W[16 nt + l%16][128 kt + 32 (l/16) + 16 h +
 * 0..15]. One wavefront therefore reads a tile with two fully coalesced 1 KiB
 * loads and each lane ends up holding the 32 consecutive K values one
 * operand of a 16x16x128 FP8 MFMA (or four 16x16x32 bf16 MFMAs) needs.
 * Scale block of one expert (fp32, padded to 256 bytes):
 *   LF_FP8_SCALE_PER_CHANNEL: s[N]
 *   LF_FP8_SCALE_BLOCK128:    s[N/128][K/128]
 * The dequantized weight is fp32(q) * s.
 */
#define LF_FP8_WEIGHT_MAGIC 0x5738464Cu /* bytes "LF8W" */
#define LF_FP8_WEIGHT_VERSION 1u
#define LF_FP8_HEADER_BYTES 256
#define LF_FP8_TILE_ROWS 16
#define LF_FP8_TILE_COLUMNS 128
#define LF_FP8_TILE_BYTES 2048
#define LF_FP8_LAYOUT_TILE16X128 1u

enum lf_fp8_scale_mode {
  LF_FP8_SCALE_PER_CHANNEL = 1,
  LF_FP8_SCALE_BLOCK128 = 2
};

typedef struct lf_fp8_weight_header {
  uint32_t magic;
  uint32_t version;
  uint32_t layout;
  uint32_t scale_mode;
  uint32_t rows;        /* N: output width */
  uint32_t columns;     /* K: input width */
  uint32_t experts;     /* 1 for a dense projection */
  uint32_t reserved;
  uint64_t tile_offset;     /* = LF_FP8_HEADER_BYTES */
  uint64_t tile_bytes;      /* per expert: N * K */
  uint64_t scale_offset;    /* = tile_offset + experts * tile_bytes */
  uint64_t scale_bytes;     /* per expert, padded to 256 */
  uint8_t padding[192];
} lf_fp8_weight_header;

/* Byte size of a weight region; LF_INVALID_ARGUMENT unless N % 16 == 0,
 * K % 128 == 0 (and N % 128 == 0 for block scales), experts >= 1. */
int32_t lunaflux_fp8_weight_region_bytes(int32_t scale_mode, int64_t rows,
                                         int64_t columns, int32_t experts,
                                         int64_t *byte_count);

/* The pre-swizzle model/device_materialize applies per tensor
 * (model/device_materialize/layout.mbt:37-93 places tensors; this fills one
 * placed region). q: E x [N, K] row-major e4m3 codes (q_bytes = E N K);
 * scales: E x the scale block above, unpadded (scale_count = E N for per
 * channel, E (N/128)(K/128) for blocks). Writes the whole region (header
 * included); LF_INVALID_ARGUMENT, with nothing read, when a count or the
 * region size does not match the shape. */
int32_t lunaflux_fp8_pack_weight(int32_t scale_mode, int64_t rows,
                                 int64_t columns, int32_t experts,
                                 const uint8_t *q, int64_t q_bytes,
                                 const float *scales, int64_t scale_count,
                                 uint8_t *region, int64_t region_bytes);
/* Inverse of the pack (tests and tooling). */
int32_t lunaflux_fp8_unpack_weight(const uint8_t *region, int64_t region_bytes,
                                   uint8_t *q, int64_t q_bytes, float *scales,
                                   int64_t scale_count);

/* ---- kernel entry points ----------------------------------------------- */
/*
 * Families (one catalog AotKernelFamily each; kernels/catalog/entry.mbt:
 * 161-219):
 *  W8A16 ("decode"): bf16 activations, e4m3 weights dequantized to bf16 in
 *    registers (exact), bf16 MFMA, fp32 accumulation, per-channel scale in
 *    the epilogue. Two forms, picked per entry by the launch geometry:
 *    one-tile (a block of waves owns one 16-column tile and splits K across
 *    its waves, partials summed in LDS) and column-group (each wave owns one
 *    16-column tile, a block several adjacent tiles over one K-slice sharing
 *    the activation slice through LDS; with more than one slice the partials
 *    are reduced in a fixed slice order by the last block of each column
 *    group through the workspace). Profiles of 65..128 rows use a third,
 *    LDS-tiled GEMM form (_m128_n64 / _m128_n128: blocks of 8 waves own
 *    128 rows x BN weight columns over a K-slice; activation and weight
 *    tiles stream global -> LDS in two rings loaded by different waves),
 *    except vocabulary-wide dense shapes. Suffix _m16/_m32/_m64/_m128: the
 *    profile's largest M; _k<K>...: a shape-specialized entry.
 *  W8A8 ("prefill"): activations quantized per token to e4m3
 *    (lf_fp8_act_quant_rows), e4m3 x e4m3 MFMA, fp32 accumulation, row scale
 *    x channel scale epilogue. _t256: 256 x 256 tiles of 4 waves
 *    (16x16x128 f8f6f4 MFMA, 128 x 128 outputs per wave) for launches of at
 *    least 256 such tiles; _t256w8: the same tiles on 8 waves (32x32x64
 *    f8f6f4 MFMA, 512-thread blocks) for 192-255; _t256x128 (QKV, dense):
 *    256 x 128 tiles of 4 waves when those number 128-256; _t128: 128 x 128
 *    tiles of 4 waves otherwise.
 *
 * Operands (all device regions, in order):
 *  lf_fp8_act_quant_rows (counts, x, w, xq)   x bf16 [M, K] -> xq; K is read
 *                                             from the header of w, the
 *                                             first weight of the op the
 *                                             quantizer feeds
 *  *_dense     (counts, x, w, y)              y bf16 [M, N]
 *  *_qkv       (counts, x, wq, wk, wv, y)     y bf16 [M, Nq+Nk+Nv] = Q|K|V
 *  *_gate_up   (counts, x, wg, wu, h)         h bf16 [M, I],
 *                                             h = silu(x Wg^T) * (x Wu^T)
 * The W8A16 forms take one more operand, ws (after y / h): the split-K
 * workspace, lunaflux_fp8_w8a16_workspace_bytes(entry, N, K, max) bytes,
 * zero-filled once when it is allocated (its arrival counters return to zero
 * at the end of every launch; launches sharing one ws must not overlap).
 * The W8A8 forms take xq (the quantizer's output) in place of x. xq layout:
 * e4m3 codes [M, K] at offset 0, fp32 row scales at offset
 * align256(M * K); its size for a profile is lunaflux_fp8_act_quant_bytes.
 * The _aq forms (below) take x and quantize it inside the same launch.
 * GatedMlp (model/plan/plan.mbt:47-59) runs as one launch
 * (lunaflux_fp8_gated_mlp_geometry: W8A16 at the Llama-3-8B widths, W8A8
 * for any width), or as gate_up into the workspace followed by dense(down)
 * from it.
 */
#define LF_FP8_COUNTS_QUERY_TOKENS 3
#define LF_FP8_COUNTS_BYTES 20
#define LF_FP8_SYMBOL_BYTES 128

int64_t lunaflux_fp8_act_quant_bytes(int64_t max_rows, int64_t columns);
/* Split-K workspace of a W8A16 entry for (N, K, max_query_tokens): fp32
 * partial tiles plus one arrival counter per column group; -1 if the shape
 * is not supported (N % 16, K % 128, max > 128). */
int64_t lunaflux_fp8_w8a16_workspace_bytes(int32_t entry, int64_t n, int64_t k,
                                           int32_t max_tokens);

enum lf_fp8_entry {
  LF_FP8_ENTRY_ACT_QUANT_ROWS = 1,
  LF_FP8_ENTRY_W8A16_DENSE = 2,
  LF_FP8_ENTRY_W8A16_QKV = 3,
  LF_FP8_ENTRY_W8A16_GATE_UP = 4,
  LF_FP8_ENTRY_W8A8_DENSE = 5,
  LF_FP8_ENTRY_W8A8_QKV = 6,
  LF_FP8_ENTRY_W8A8_GATE_UP = 7,
  LF_FP8_ENTRY_RMS_NORM_QUANT_ROWS = 8,
  LF_FP8_ENTRY_GROUPED = 9, /* admission only: the MoE expert weights */
  LF_FP8_ENTRY_W8A16_GATED_MLP = 10,
  /* W8A8 operations as one launch each, the per-token quantizer inside */
  LF_FP8_ENTRY_W8A8_DENSE_AQ = 11,
  LF_FP8_ENTRY_W8A8_QKV_AQ = 12,
  LF_FP8_ENTRY_W8A8_GATE_UP_AQ = 13,
  LF_FP8_ENTRY_W8A8_GATED_MLP = 14,
  /* Weights with 128 x 128 block scales (LF_FP8_SCALE_BLOCK128), below */
  LF_FP8_ENTRY_W8A16_DENSE_B128 = 15,
  LF_FP8_ENTRY_W8A16_QKV_B128 = 16,
  LF_FP8_ENTRY_W8A16_GATE_UP_B128 = 17,
  LF_FP8_ENTRY_W8A8_DENSE_B128 = 18,
  LF_FP8_ENTRY_W8A8_QKV_B128 = 19,
  LF_FP8_ENTRY_W8A8_GATE_UP_B128 = 20,
  LF_FP8_ENTRY_W8A8_GATED_MLP_B128 = 21,
  LF_FP8_ENTRY_W8A16_GATED_MLP_B128 = 22
};

/* Block-scaled projections (checkpoints whose weights carry weight_scale_inv
 * 128 x 128 block scales: W = q s[n / 128][k / 128]); N and K multiples of
 * 128, every Q / K / V width of a QKV operation too.
 *  W8A16: lf_fp8_w8a16_{dense,qkv,gate_up}_b128_m{16,32,64,128} and, for
 *      profiles of 65..128 rows, lf_fp8_w8a16_{op}_b128_m128_n{64,128}
 *      (the per-channel entry's LDS-tiled GEMM geometry rule, except that
 *      at equal block counts it takes BN 128 where the per-channel entry
 *      takes BN 64); operands and
 *      workspace as the per-channel W8A16 entries
 *      (lunaflux_fp8_w8a16_workspace_bytes with the _B128 entry); each
 *      k-tile's products scaled by its block scale:
 *      y = sum_kt s[n / 128][kt] sum_{k in kt} x_k q_nk.
 *  W8A8: lf_fp8_w8a8_{dense,qkv,gate_up}_b128 (counts, x, w..., y, ws), one
 *      launch each: x quantized per token per 128-column group (amax over
 *      the group, the per-token quantizer's arithmetic) inside the launch,
 *      then y = sum_kt sa[m][kt] s[n / 128][kt] sum_{k in kt} qa_mk q_nk on
 *      256-row bands: lf_fp8_w8a8_{op}_b128_t256 (256 x 256 tiles, from 192
 *      such tiles on; widths multiples of 256, gate/up: of 128) or
 *      lf_fp8_w8a8_{op}_b128_t256x128 (256 x 128 tiles), 512 threads; for
 *      K >= 2^24 lf_fp8_w8a8_{op}_b128 on 128 x 128 tiles (256 threads,
 *      128-row bands). ws: lunaflux_fp8_w8a8_workspace_bytes with the _B128
 *      entry (it follows the form), error word at LF_FP8_AQ_ERROR_OFFSET as
 *      for the _AQ entries.
 *      lf_fp8_w8a8_gated_mlp_b128 (counts, x, wg, wu, wd, y, ws): GatedMlp
 *      in one launch (group quantizer, gate/up + SwiGLU, group quantizer of
 *      h, down), lunaflux_fp8_gated_mlp_geometry / _workspace_bytes with
 *      LF_FP8_ENTRY_W8A8_GATED_MLP_B128; lf_fp8_w8a8_gated_mlp_b128_t256
 *      (the same operands, 512 threads) on 256 x 256 tiles where the
 *      gate/up launch takes them and the hidden width is a multiple of 256.
 *  W8A16 shape-specialized (Llama-3-8B widths, profiles of <= 32 rows, as
 *      the per-channel ones): lf_fp8_w8a16_{dense,gate_up}_b128_k{K}_mM,
 *      lf_fp8_w8a16_qkv_b128_k4096_q4096_kv1024_mM (picked by
 *      lunaflux_fp8_qkv_launch_geometry; without the split,
 *      lunaflux_fp8_w8a16_workspace_bytes sizes the QKV_B128 workspace for
 *      every entry of that width). W8A16 GatedMlp in one launch with
 *      LF_FP8_ENTRY_W8A16_GATED_MLP_B128 (the per-channel one-launch forms:
 *      lf_fp8_w8a16_gated_mlp_b128_h4096_i14336_m{16,32} and
 *      lf_fp8_w8a16_gated_mlp_b128_m128_n128_n{64,128}; workspace and error
 *      word as LF_FP8_ENTRY_W8A16_GATED_MLP).
 * The geometry functions take the _B128 entries as the per-channel ones;
 * admission requires block scales for them (and channel scales for every
 * other dense entry). */

/* One launch per W8A8 operation (the plan binds one AOT entry point per
 * operation, kernels/launch_contract/types.mbt:16-27, and rejects a second
 * contract for the same (profile, operation), paged_admit.mbt:275-279):
 *  lf_fp8_w8a8_{dense,qkv,gate_up}_{t256,t256x128,t256w8,t128}_aq
 *      (counts, x, w..., y, ws)   operands as the W8A16 forms: x bf16 [M, K]
 * The grid's first 256 blocks quantize x per token (the codes and scales of
 * lf_fp8_act_quant_rows) into ws; the GEMM's tiles follow, each starting
 * once every row of its band is quantized (counted, bounded waits: see the
 * error word below). Same outputs as the act-quant launch followed by the
 * GEMM-only entry of the same tile form. Geometry and symbol from
 * lunaflux_fp8_launch_geometry / lunaflux_fp8_qkv_launch_geometry with the
 * _AQ entry; ws: lunaflux_fp8_w8a8_workspace_bytes bytes (-1 if the shape
 * has no form), zero-filled once when allocated.
 * Workspace of every one-launch entry with counted waits (these and the
 * W8A8 GatedMlp): it starts with a sync area whose first int32 is the error
 * word, 0 after every correct launch; 1 if a wait ran out (never on a
 * correct launch; the polls are bounded, so no launch hangs). Once it is
 * set, launches on that workspace leave their outputs unwritten until the
 * caller zero-fills the workspace again (its counters are then not at
 * rest).
 * Launches sharing one ws must not overlap. */
#define LF_FP8_AQ_ERROR_OFFSET 0
int64_t lunaflux_fp8_w8a8_workspace_bytes(int32_t entry, int64_t n, int64_t k, int32_t max_tokens);

/* Admission of one weight operand's region before an operation is bound,
 * the FP8 counterpart of the exact BF16 size check engine/device_plan applies
 * to every weight region (build.mbt:149-203). region_head: the region's
 * first LF_FP8_HEADER_BYTES (the header the pack wrote, kept by the
 * materializer); region_bytes: the TensorRef region's size. The header must
 * carry the format's magic, version and layout, the shape (rows = N,
 * columns = K, experts; 1 for the dense families) and the format's own
 * offsets, and region_bytes must equal lunaflux_fp8_weight_region_bytes for
 * it. LF_UNSUPPORTED for a valid region whose scale mode is not the
 * entry's: block scales on a per-channel dense, QKV, gate/up or GatedMlp
 * entry (their kernels read one scale per output channel), channel scales
 * on a _B128 entry (LF_FP8_ENTRY_GROUPED admits both);
 * LF_INVALID_ARGUMENT for anything else that does not hold. The
 * shape-specialized W8A16 entries start streaming weights before they read
 * the header, so this check is what bounds their reads. */
int32_t lunaflux_fp8_admit_weight(int32_t entry, const uint8_t *region_head,
                                  int64_t head_bytes, int64_t region_bytes,
                                  int64_t rows, int64_t columns,
                                  int32_t experts);

/* Launch geometry a manifest records for (entry, output width N, input width
 * K, profile max_query_tokens): grid xyz, block xyz, dynamic LDS bytes and
 * the symbol to load (NUL-terminated, <= 128 bytes). For _QKV, N is the
 * packed width Nq + Nk + Nv; for _GATE_UP, N is the intermediate width I. */
int32_t lunaflux_fp8_launch_geometry(int32_t entry, int64_t n, int64_t k,
                                     int32_t max_tokens, int32_t dims[7],
                                     char symbol[LF_FP8_SYMBOL_BYTES]);

/* W8A16 profiles with max_query_tokens <= 32 select a shape-specialized
 * entry (K, and for QKV the Q / K-V split, compiled into the symbol, e.g.
 * lf_fp8_w8a16_gate_up_k4096_m32) where one is built, like an AOT kernel
 * compiled for one model shape; other shapes use the generic entries. A
 * specialized entry checks the weight header against its compiled shape and
 * leaves the output unwritten on a mismatch. The QKV split is not
 * recoverable from N alone, so QKV operations call these variants with
 * Nq and Nk = Nv (the catalog records the split of the model's layer); the
 * plain functions above pick the generic QKV entry. */
int32_t lunaflux_fp8_qkv_launch_geometry(int32_t entry, int64_t nq, int64_t nkv, int64_t k,
                                         int32_t max_tokens, int32_t dims[7],
                                         char symbol[LF_FP8_SYMBOL_BYTES]);
int64_t lunaflux_fp8_qkv_w8a16_workspace_bytes(int64_t nq, int64_t nkv, int64_t k,
                                               int32_t max_tokens);

/* GatedMlp in one launch (model/plan/plan.mbt:47-59: one operation of arity
 * (4, 1); kernels/reference/mlp.mbt:4-39), W8A16, built for the Llama-3-8B
 * widths (H = 4096, I = 14336) and profiles of <= 16 and <= 32 rows:
 *  lf_fp8_w8a16_gated_mlp_h4096_i14336_m16 / _m32
 *      (counts, x, wg, wu, wd, y, ws)   x, y bf16 [M, H]
 * The same arithmetic as the W8A16 gate_up launch (h rounded to bf16) then
 * the dense(down) launch: the grid's first blocks compute h into ws, the
 * others the down projection, each down K-slice starting once the blocks
 * writing its h columns have counted themselves done (bounded polls that
 * cannot hang; a poll that ran out sets the int32 error word at ws + size -
 * LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END, never on a correct launch, and
 * the word stays set). ws: lunaflux_fp8_gated_mlp_workspace_bytes bytes,
 * zero-filled once when allocated (its counters return to zero at the end
 * of every launch; launches sharing one ws must not overlap). Geometry and
 * symbol from lunaflux_fp8_gated_mlp_geometry, which returns LF_UNSUPPORTED
 * for shapes or profiles without an entry: the operation then runs as the
 * gate_up and dense launches. Weights are admitted as for the dense entries
 * (entry LF_FP8_ENTRY_W8A16_GATED_MLP, per-channel scales). On MI355X the
 * two launches are faster (38.6 vs 44.8 us at M = 32: back-to-back launches
 * cost little, and the down blocks learn that h is complete 3-5 us after the
 * last gate/up block counts itself), so this entry is for callers that need
 * the operation as a single launch. */
#define LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END 128
/* With entry LF_FP8_ENTRY_W8A8_GATED_MLP (any H, I that are multiples of
 * 128, any profile): the W8A8 GatedMlp in one launch,
 *  lf_fp8_w8a8_gated_mlp_{t256_t256,t256_t256x128,t128_t128}
 *      (counts, x, wg, wu, wd, y, ws)   x, y bf16 [M, H]
 * the act-quant, gate/up (SwiGLU, h rounded to bf16), act-quant of h and
 * down launches as four counted steps of one grid (gate/up and down tile
 * forms in the name), with the same outputs. ws as for the _AQ entries
 * (error word at offset LF_FP8_AQ_ERROR_OFFSET), sized by
 * lunaflux_fp8_gated_mlp_workspace_bytes with this entry. */
int32_t lunaflux_fp8_gated_mlp_geometry(int32_t entry, int64_t hidden, int64_t inter,
                                        int32_t max_tokens, int32_t dims[7],
                                        char symbol[LF_FP8_SYMBOL_BYTES]);
int64_t lunaflux_fp8_gated_mlp_workspace_bytes(int32_t entry, int64_t hidden, int64_t inter,
                                               int32_t max_tokens);

/* RmsNorm fused with the per-token quantizer: the RmsNorm operation
 * (kernels/reference/basic.mbt:32-68; catalog capability rms_norm,
 * kernels/catalog/entry.mbt:60,79) writing its output as the xq region the
 * W8A8 projection after it reads, in place of a bf16 activation plus an
 * lf_fp8_act_quant_rows launch.
 *  lf_fp8_rms_norm_quant_rows_eps1em5 / _eps1em6
 *      (counts, x, g, w, xq)   x bf16 [M, K]; g bf16 [K] (the norm weight's
 *                              TensorRef region); w the first weight of the
 *                              projection fed (K is read from its header,
 *                              K <= 8192); xq as for lf_fp8_act_quant_rows.
 * Per row: inv = 1 / sqrt(sum_k x^2 / K + eps), y = (x * inv) * g in fp32,
 * then the quantizer's codes and scale of y. The sum of squares is reduced
 * across a wavefront (not the reference's sequential order), so results
 * match the reference to fp32 rounding of inv, not bit for bit.
 * The epsilon is part of the operation shape (model/plan/plan.mbt:146-151),
 * so each value is its own entry: geometry and symbol for (epsilon, K,
 * max_rows); LF_UNSUPPORTED for an epsilon with no entry (1e-5 and 1e-6 as
 * fp32 are built). lunaflux_fp8_launch_geometry rejects this entry
 * (LF_INVALID_ARGUMENT), as it carries no epsilon. */
int32_t lunaflux_fp8_rms_norm_quant_geometry(float epsilon, int64_t k, int32_t max_rows,
                                             int32_t dims[7],
                                             char symbol[LF_FP8_SYMBOL_BYTES]);

/* ---- grouped form: MoE expert MLP ---------------------------------------- */
/*
 * The reference has no MoE (its plan vocabulary stops at GatedMlp,
 * model/plan/operations.mbt:4-14), so these entry points define the operand
 * lists a MoE operation would bind. Expert weights are weight regions with
 * `experts` = E: gate and up [E][I, H], down [E][H, I]; per-channel scales
 * with per-token activation quantization (group 0), or 128 x 128 block scales
 * with per-token-per-128-column activation quantization (group 128).
 *
 * The routing descriptor is a 32-byte device region (a model constant, like
 * a weight) read by every MoE kernel. The workspace is one region whose
 * layout is a function of the live token count (the counts descriptor) and
 * the routing descriptor; lunaflux_fp8_moe_workspace_bytes sizes it for a
 * profile's max_query_tokens.
 *
 * Launch sequence and operands (in order):
 *  lf_moe_route[_sort]  (counts, desc, logits fp32 [T, E], x bf16 [T, H], ws)
 *  lf_moe_sort_count    (counts, desc, ws)    (not after lf_moe_route_sort)
 *  lf_moe_sort          (counts, desc, ws)    (not after lf_moe_route_sort)
 *  lf_moe_quant_tokens  (counts, desc, x bf16 [T, H], ws)  (not after lf_moe_route_sort)
 * (lf_moe_route_sort: routing, the whole sort and the token quantizer in one
 * 1024-thread block, chosen for profiles of max_tokens * top_k <= 1024; the
 * geometry then returns LF_OK with an empty symbol and zero dims for
 * LF_FP8_MOE_SORT_COUNT, LF_FP8_MOE_SORT and LF_FP8_MOE_QUANT_TOKENS,
 * meaning no launch. Its outputs equal those of the four launches.
 * lf_moe_route does not read x.)
 *  lf_moe_gate_up[_b128|_t256|_t256_b128_q|_gemv](counts, desc, wg, wu, ws)
 *  lf_moe_quant_hidden  (counts, desc, ws)    (not with _t256_b128_q or _t256_aq)
 *  lf_moe_down[_b128|_t256_b128|_gemv]   (counts, desc, wd, ws)
 *  lf_moe_down_t256_aq  (counts, desc, wd, ws, sync)
 * (_t256_aq: per-channel profiles on 256-row tiles; the hidden quantizer
 * runs as the first counted step of the down launch: 256 blocks quantize h
 * per token (the codes and scales of lf_moe_quant_hidden) and each down tile
 * starts once every row of its 256-row tile is quantized, so the geometry
 * gives LF_FP8_MOE_QUANT_HIDDEN no launch. sync: the region of the
 * workspace from lunaflux_fp8_moe_sync_offset to its end, zero-filled once
 * when allocated (its counters return to zero at the end of every launch;
 * launches sharing one workspace must not overlap); its first int32 is the
 * error word of the one-launch entries, LF_FP8_AQ_ERROR_OFFSET.)
 * (_t256: the GEMMs on 256 x 256 tiles, chosen by the launch geometry for
 * profiles that average >= 256 routed rows per expert, _t256_b128 with block
 * scales where both GEMMs have K <= 3072, its gate/up as _t256_b128_q, whose
 * epilogue also runs the hidden quantizer (a block's 128 h-columns are one
 * scale group): lunaflux_fp8_moe_launch_geometry then returns LF_OK with an
 * empty symbol and zero dims for LF_FP8_MOE_QUANT_HIDDEN, meaning no launch;
 * _gemv:
 * either scale mode, chosen for profiles of at most 32 tokens, where the
 * GEMMs stream the touched experts' weights: a fixed grid whose blocks
 * loop over (expert with rows, 64-column group) items.
 * With per-token scales lf_moe_quant_tokens reads the sort's positions and
 * also writes each token's scale in expert order, so it runs after
 * lf_moe_sort.)
 *  lf_moe_combine       (counts, desc, ws, out bf16 [T, H])
 * Routing: the k largest logits per token (ties to the lower expert id);
 * weights are a softmax over the k picked logits (route_mode 0, Mixtral) or
 * the softmax over all experts at the picked ids (route_mode 1). The sort is
 * a stable counting sort of assignments a = t*k + j by expert; out[t] =
 * sum_j w[t, j] * y(t, j) in ascending j, fp32, rounded to bf16.
 */
#define LF_FP8_MOE_MAGIC 0x454F4D4Cu /* bytes "LMOE" */

typedef struct lf_fp8_moe_desc {
  uint32_t magic;
  int32_t experts;
  int32_t top_k;
  int32_t route_mode;
  int32_t hidden;
  int32_t inter;
  int32_t group; /* 0: per token / per channel; 128: 128-wide blocks */
  int32_t reserved;
} lf_fp8_moe_desc;

enum lf_fp8_moe_entry {
  LF_FP8_MOE_ROUTE = 1,
  LF_FP8_MOE_SORT = 2,
  LF_FP8_MOE_QUANT_TOKENS = 3,
  LF_FP8_MOE_GATE_UP = 4,
  LF_FP8_MOE_QUANT_HIDDEN = 5,
  LF_FP8_MOE_DOWN = 6,
  LF_FP8_MOE_COMBINE = 7,
  LF_FP8_MOE_SORT_COUNT = 8 /* runs between ROUTE and SORT */
};

/* Validates and fills a descriptor: 1 <= experts <= 256, 1 <= top_k <=
 * min(experts, 16), route_mode 0 or 1, hidden and inter multiples of 128,
 * group 0 or 128 (128 also needs hidden, inter <= 4096). */
int32_t lunaflux_fp8_moe_descriptor(int32_t experts, int32_t top_k,
                                    int32_t route_mode, int64_t hidden,
                                    int64_t inter, int32_t group,
                                    lf_fp8_moe_desc *out);
/* Workspace bytes for up to max_tokens live tokens (the arrays below for
 * max_tokens, then the down launch's counter area where it takes one); -1 if
 * invalid. */
int64_t lunaflux_fp8_moe_workspace_bytes(const lf_fp8_moe_desc *desc,
                                         int32_t max_tokens);
/* Byte offset of the counter area (sync operand of lf_moe_down_t256_aq)
 * inside that workspace: the end of the arrays for max_tokens, so no live
 * token count moves it; -1 if the profile's down entry takes none. */
int64_t lunaflux_fp8_moe_sync_offset(const lf_fp8_moe_desc *desc, int32_t max_tokens);
/* Byte offsets of the workspace arrays for `tokens` live tokens, in order:
 * top-k ids (int32 [T*k]), top-k weights (fp32 [T*k]), sorted assignments
 * (int32 [T*k]), position of each assignment (int32 [T*k]), expert row
 * offsets (int32 [E+1]), expert 128-row tile offsets (int32 [E+1]) followed
 * by the 256-row tile offsets (int32 [E+1]), the number of experts with rows
 * (int32) and their ids ascending (int32 [E]), e4m3
 * tokens [T, H], token scales, h bf16 [T*k, I], e4m3 h, h scales, y bf16
 * [T*k, H], end. */
int32_t lunaflux_fp8_moe_workspace_layout(const lf_fp8_moe_desc *desc,
                                          int32_t tokens, int64_t offsets[13]);
int32_t lunaflux_fp8_moe_launch_geometry(int32_t entry,
                                         const lf_fp8_moe_desc *desc,
                                         int32_t max_tokens, int32_t dims[7],
                                         char symbol[LF_FP8_SYMBOL_BYTES]);

#ifdef __cplusplus
}
#endif

#endif
