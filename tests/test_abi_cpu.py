"""CPU tests of the C-ABI library: it loads, exports every function the
headers declare, and its host-side pieces (weight pre-swizzle, region sizes,
launch geometry, argument validation) behave as documented. No kernel runs.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_lib as o
from lunaflux_amd import _abi, fp8, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for header in ("lunaflux_hip.h", "lunaflux_fp8.h"):
        text = open(os.path.join(ROOT, "include", header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(lunaflux_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_abi.LIBRARY_PATH)
    names = declared_functions()
    assert len(names) >= 38
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing
    # and the Python binding declares each of them
    assert set(names) == set(_abi.SIGNATURES)


def test_code_object_has_every_entry_point():
    image = _abi.code_object_bytes()
    for symbol in ["lf_fp8_act_quant_rows"] + [f"lf_fp8_w8a8_{op}_{t}" for op in ("dense", "qkv", "gate_up")
                                               for t in ("t128", "t256", "t256w8", "t256x128")] + ["lf_moe_route", "lf_moe_route_sort", "lf_moe_sort_count", "lf_moe_sort", "lf_moe_quant_tokens",
                   "lf_moe_gate_up", "lf_moe_gate_up_b128", "lf_moe_quant_hidden", "lf_moe_down",
                   "lf_moe_down_b128", "lf_moe_combine", "lf_moe_gate_up_gemv", "lf_moe_down_gemv",
                   "lf_moe_gate_up_t256_b128", "lf_moe_down_t256_b128", "lf_moe_down_t256_aq"] + [f"lf_fp8_w8a16_{op}_m{m}" for op in ("dense", "qkv", "gate_up")
                                             for m in (16, 32, 64, 128)] + [
                   f"lf_fp8_w8a16_{op}_m16_t1" for op in ("dense", "qkv", "gate_up")] + [
                   f"lf_fp8_w8a16_dense_k{k}_m{m}" for k in (4096, 14336) for m in (16, 32)] + [
                   f"lf_fp8_w8a16_gate_up_k4096_m{m}" for m in (16, 32)] + [
                   f"lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m{m}" for m in (16, 32)] + [
                   f"lf_fp8_w8a16_{op}_m128_n{bn}" for op in ("dense", "qkv", "gate_up") for bn in (64, 128)] + [
                   f"lf_fp8_w8a16_dense_wide_k4096_m{m}" for m in (16, 32, 128)] + [
                   "lf_fp8_rms_norm_quant_rows_eps1em5", "lf_fp8_rms_norm_quant_rows_eps1em6"] + [
                   f"lf_fp8_w8a16_{op}_b128_m{m}" for op in ("dense", "qkv", "gate_up") for m in (16, 32, 64, 128)] + [
                   f"lf_fp8_w8a8_{op}_b128" for op in ("dense", "qkv", "gate_up", "gated_mlp")]:
        assert symbol.encode() + b"\0" in image, symbol


def test_probe_without_gpu_is_an_availability_code():
    out = (ctypes.c_int64 * 3)()
    availability = _abi.lib().lunaflux_hip_probe(out)
    assert availability in range(0, 7)
    assert out[2] == 0  # no vendor GEMM


def test_swizzle_matches_documented_layout():
    rng = np.random.default_rng(1)
    n, k = 48, 384
    q = rng.integers(0, 256, (n, k), dtype=np.uint8)
    s = rng.random(n, dtype=np.float32)
    region = fp8.pack_weight(q, s)
    head = region[:64]
    h32 = head.view(np.uint32)
    assert h32[0] == 0x5738464C and bytes(head[:4]) == b"LF8W"
    assert list(h32[1:8]) == [1, 1, 1, n, k, 1, 0]
    h64 = head[32:64].view(np.uint64)
    assert list(h64) == [256, n * k, 256 + n * k, (n * 4 + 255) // 256 * 256]
    assert region.size == 256 + n * k + (n * 4 + 255) // 256 * 256
    tiles = region[256:256 + n * k]
    # W[16 nt + l%16][128 kt + 32 (l/16) + 16 h + b] at tile*2048 + h*1024 + l*16 + b
    for (row, col) in [(0, 0), (17, 5), (47, 383), (31, 200), (5, 130)]:
        nt, r = divmod(row, 16)
        kt, kk = divmod(col, 128)
        g, rem = divmod(kk, 32)
        h, b = divmod(rem, 16)
        lane = g * 16 + r
        off = (nt * (k // 128) + kt) * 2048 + h * 1024 + lane * 16 + b
        assert tiles[off] == q[row, col]
    np.testing.assert_array_equal(region[256 + n * k:256 + n * k + 4 * n].view(np.float32), s)
    q2, s2, info = fp8.unpack_weight(region)
    np.testing.assert_array_equal(q2[0], q)
    np.testing.assert_array_equal(s2[0], s)


def test_pack_experts_and_block_scales():
    rng = np.random.default_rng(2)
    q = rng.integers(0, 256, (3, 128, 256), dtype=np.uint8)
    s = rng.random((3, 2), dtype=np.float32)
    region = fp8.pack_weight(q, s, fp8.BLOCK128)
    q2, s2, info = fp8.unpack_weight(region)
    assert info == dict(scale_mode=2, rows=128, columns=256, experts=3)
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_array_equal(s2, s)


def test_region_size_validation():
    for rows, cols, mode in [(15, 128, 1), (16, 100, 1), (16, 128, 2), (0, 128, 1), (16, 128, 9)]:
        with pytest.raises(fp8.DeviceError):
            fp8.weight_region_bytes(rows, cols, 1, mode)


def test_launch_geometry():
    # W8A16 generic forms, max rows <= 16: one 16-column tile per 8-wave
    # block, K split across its waves. Larger profiles: 4 column tiles per
    # 4-wave block, K cut into about 512 / groups slices across blocks.
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 2048, 32)
    assert sym == "lf_fp8_w8a16_dense_m32" and dims.grid == (64 * 8, 1, 1) and dims.block == (256, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, 6144, 4096, 1)
    assert sym == "lf_fp8_w8a16_qkv_m16_t1" and dims.grid == (384, 1, 1) and dims.block == (512, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, 14336, 2048, 32)
    assert sym == "lf_fp8_w8a16_gate_up_m32" and dims.grid == (224 * 2, 1, 1)
    # 65..128 rows, N not a multiple of 64: the generic column-group form
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, 6160, 4096, 128)
    assert sym == "lf_fp8_w8a16_qkv_m128" and dims.grid == (97 * 5, 1, 1)
    # split-K workspace: S x (N / 16) x NW x MT 1 KiB fragments + one counter
    # per column group; 256 bytes (unused) without a split
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_DENSE, 4096, 2048, 32) == 8 * 256 * 2 * 1024 + 256
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_QKV, 6144, 4096, 1) == 256
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_GATE_UP, 14336, 2048, 32) == 2 * 896 * 2 * 2 * 1024 + 1024
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_QKV, 6144, 4096, 128) == 2 * 96 * 8 * 4 * 1024 + 512
    # Shape-specialized (Llama-3-8B) entries for profiles of <= 32 rows.
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 14336, 32)
    assert sym == "lf_fp8_w8a16_dense_k14336_m32" and dims.grid == (64 * 4, 1, 1)
    assert dims.block == (256, 1, 1)
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_DENSE, 4096, 14336, 32) == 4 * 256 * 2 * 1024 + 256
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 4096, 8)
    assert sym == "lf_fp8_w8a16_dense_k4096_m16" and dims.grid == (256, 1, 1) and dims.block == (512, 1, 1)
    # gate/up: unsplit column groups (4 tiles per block at 32 rows, 2 at 16)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, 14336, 4096, 32)
    assert sym == "lf_fp8_w8a16_gate_up_k4096_m32" and dims.grid == (224, 1, 1)
    assert dims.block == (256, 1, 1)
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_GATE_UP, 14336, 4096, 32) == 256
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, 14336, 4096, 16)
    assert sym == "lf_fp8_w8a16_gate_up_k4096_m16" and dims.grid == (448, 1, 1)
    assert dims.block == (128, 1, 1)
    # QKV at 32 rows: 8 tiles per block over 4 K-slices (48 groups x 4)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, 6144, 4096, 32, qkv_split=(4096, 1024))
    assert sym == "lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m32" and dims.grid == (192, 1, 1)
    assert dims.block == (512, 1, 1)
    assert (fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_QKV, 6144, 4096, 32, (4096, 1024))
            == 4 * 384 * 2 * 1024 + 256)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, 6144, 4096, 16, qkv_split=(4096, 1024))
    assert sym == "lf_fp8_w8a16_qkv_k4096_q4096_kv1024_m16" and dims.grid == (384, 1, 1)
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_QKV, 6144, 4096, 16, (4096, 1024)) == 256
    # a QKV split without an entry, or a profile above 32 rows: generic
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, 6144, 4096, 32, qkv_split=(2048, 2048))
    assert sym == "lf_fp8_w8a16_qkv_m32"
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 4096, 64)
    assert sym == "lf_fp8_w8a16_dense_m64"
    # 65..128 rows: the LDS-tiled GEMM, 128 x BN tiles (gate/up blocks cover
    # BN / 2 h-columns): among BN 64 / 128 and the splits keeping >= 8
    # k-tiles per slice, the most blocks up to 256, the smaller split on a
    # tie; with more than 256 column blocks unsplit, BN 128 unsplit
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 4096, 128)
    assert sym == "lf_fp8_w8a16_dense_m128_n64" and dims.grid == (64 * 4, 1, 1)
    assert dims.block == (512, 1, 1)
    # S x blocks x 8 waves x (2 x BN / 32) 1 KiB fragments + a counter per block
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_DENSE, 4096, 4096, 128) == 4 * 64 * 8 * 4 * 1024 + 256
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 14336, 100)
    assert sym == "lf_fp8_w8a16_dense_m128_n64" and dims.grid == (64 * 4, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_QKV, 6144, 4096, 128, qkv_split=(4096, 1024))
    assert sym == "lf_fp8_w8a16_qkv_m128_n64" and dims.grid == (96 * 2, 1, 1)
    # (a tie: BN 128 x 2 slices and BN 64 unsplit both give 256 blocks)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, 8192, 2048, 128)
    assert sym == "lf_fp8_w8a16_gate_up_m128_n64" and dims.grid == (256, 1, 1)
    # more than 256 column blocks even unsplit: BN 128, no split
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 40960, 1024, 128)
    assert sym == "lf_fp8_w8a16_dense_m128_n128" and dims.grid == (320, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_GATE_UP, 14336, 4096, 128)
    assert sym == "lf_fp8_w8a16_gate_up_m128_n128" and dims.grid == (224, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 2048, 65)
    assert sym == "lf_fp8_w8a16_dense_m128_n64" and dims.grid == (64 * 2, 1, 1)  # 16 k-tiles
    # wide dense shapes (N >= 16384, e.g. the 128,256-column vocabulary head)
    for mt, w in ((16, 2), (32, 4), (128, 8)):
        dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 128256, 4096, mt)
        assert sym == f"lf_fp8_w8a16_dense_wide_k4096_m{mt}" and dims.grid == (8016 // w, 1, 1)
        assert dims.block == (64 * w, 1, 1)
        assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_DENSE, 128256, 4096, mt) == 256
    assert fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 16368, 4096, 32)[1] == "lf_fp8_w8a16_dense_k4096_m32"
    assert fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_GATE_UP, 14336, 4096, 128) == 256
    # the W8A8 QKV split variant picks the same entry as the plain call
    assert (fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 2048, qkv_split=(4096, 1024))[1]
            == fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 2048)[1])
    with pytest.raises(fp8.DeviceError):
        fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A8_DENSE, 4096, 4096, 16)
    # W8A8: 256 x 256 tiles (1-D grid) from 192 of them (3/4 of a tile per
    # CU), on 8 waves below 256 tiles and on 4 waves from there; below 192,
    # QKV and dense on 256 x 128 tiles when they number 128-256, else 128 x
    # 128 tiles (4 waves), as when N does not divide.
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 2048)
    assert sym == "lf_fp8_w8a8_qkv_t256w8" and dims.grid == (8 * 24, 1, 1) and dims.block == (512, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 2560)
    assert sym == "lf_fp8_w8a8_qkv_t256w8" and dims.grid == (10 * 24, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 8192, 4096, 2048)
    assert sym == "lf_fp8_w8a8_qkv_t256" and dims.grid == (8 * 32, 1, 1) and dims.block == (256, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 4096, 4096, 2048)
    assert sym == "lf_fp8_w8a8_dense_t256x128" and dims.grid == (8 * 32, 1, 1) and dims.block == (256, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 1024)
    assert sym == "lf_fp8_w8a8_qkv_t256x128" and dims.grid == (4 * 48, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 1536)   # 288 such tiles
    assert sym == "lf_fp8_w8a8_qkv_t128" and dims.grid == (12 * 48, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 4096, 4096, 512)    # 64 such tiles
    assert sym == "lf_fp8_w8a8_dense_t128" and dims.grid == (4 * 32, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_GATE_UP, 14336, 4096, 256)  # never on 256 x 128
    assert sym == "lf_fp8_w8a8_gate_up_t128" and dims.grid == (2 * 224, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_GATE_UP, 14336, 4096, 8192)
    assert sym == "lf_fp8_w8a8_gate_up_t256" and dims.grid == (32 * 112, 1, 1) and dims.block == (256, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 4096, 14336, 2048)
    assert sym == "lf_fp8_w8a8_dense_t256x128" and dims.grid == (8 * 32, 1, 1) and dims.block == (256, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV, 6144, 4096, 8000)
    assert sym == "lf_fp8_w8a8_qkv_t256" and dims.grid == (32 * 24, 1, 1)
    dims, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 128 * 33, 4096, 8192)
    assert sym == "lf_fp8_w8a8_dense_t128" and dims.grid == (64 * 33, 1, 1)
    # the four-wave forms take 32-bit activation offsets from a tile's first
    # row (256 K < 2^32), as does the eight-wave form: from K = 2^24 the
    # 128 x 128 form
    big_k = 1 << 24
    assert fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 8192, big_k - 128, 2048)[1] == "lf_fp8_w8a8_dense_t256"
    assert fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 8192, big_k - 128, 1536)[1] == "lf_fp8_w8a8_dense_t256w8"
    for n, m in ((8192, 2048), (8192, 1536), (4096, 2048)):
        assert fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, n, big_k, m)[1] == "lf_fp8_w8a8_dense_t128"
    dims, sym = fp8.launch_geometry(_abi.ENTRY_ACT_QUANT_ROWS, 4096, 4096, 2048)
    assert sym == "lf_fp8_act_quant_rows" and dims.grid == (2048 // 4, 1, 1)  # one wave per row
    with pytest.raises(fp8.DeviceError):
        fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 4096, 129)
    with pytest.raises(fp8.DeviceError):
        fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE, 4000, 4096, 64)
    assert fp8.act_quant_bytes(3, 512) == 1536 + 256


def test_one_launch_w8a8_geometry_and_workspace():
    """The _aq entries: the GEMM-only entry's tile form, 256 quantizer blocks
    ahead of its tiles, workspace = sync area (128 B + one counter per row
    band, 256-aligned) + the quantized rows of ceil(max / BM) BM-row bands.
    The W8A8 GatedMlp: both GEMMs on 4-wave blocks of one band height."""
    for entry, plain, n, k, m in [
        (_abi.ENTRY_W8A8_DENSE_AQ, _abi.ENTRY_W8A8_DENSE, 4096, 4096, 8192),
        (_abi.ENTRY_W8A8_DENSE_AQ, _abi.ENTRY_W8A8_DENSE, 4096, 14336, 2048),
        (_abi.ENTRY_W8A8_GATE_UP_AQ, _abi.ENTRY_W8A8_GATE_UP, 14336, 4096, 8192),
        (_abi.ENTRY_W8A8_GATE_UP_AQ, _abi.ENTRY_W8A8_GATE_UP, 14336, 4096, 256),
        (_abi.ENTRY_W8A8_DENSE_AQ, _abi.ENTRY_W8A8_DENSE, 4096, 4096, 3),
    ]:
        d0, s0 = fp8.launch_geometry(plain, n, k, m)
        d1, s1 = fp8.launch_geometry(entry, n, k, m)
        assert s1 == s0 + "_aq" and d1.grid == (d0.grid[0] + 256, 1, 1) and d1.block == d0.block
        bm = 128 if s0.endswith("_t128") else 256
        bands = -(-m // bm)
        sync = 256 + 128 * bands      # error, done, one 128-byte line per band counter
        cap = bands * bm
        assert fp8.w8a8_workspace_bytes(entry, n, k, m) == sync + fp8.act_quant_bytes(cap, k)
    d, s = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV_AQ, 6144, 4096, 2048, qkv_split=(4096, 1024))
    assert s == "lf_fp8_w8a8_qkv_t256w8_aq" and d.grid == (8 * 24 + 256, 1, 1) and d.block == (512, 1, 1)
    with pytest.raises(fp8.DeviceError):
        fp8.w8a8_workspace_bytes(_abi.ENTRY_W8A8_DENSE, 4096, 4096, 16)    # the GEMM-only entry
    lib = _abi.lib()
    for h, i, m, sym, bands, gx in [
        (4096, 14336, 8192, "lf_fp8_w8a8_gated_mlp_t256_t256", 32, 112 + 16),
        (4096, 14336, 2048, "lf_fp8_w8a8_gated_mlp_t256_t256x128", 8, 112 + 32),
        (4096, 14336, 3072, "lf_fp8_w8a8_gated_mlp_t256_t256", 12, 112 + 16),    # down t256w8 alone
        (4096, 14336, 512, "lf_fp8_w8a8_gated_mlp_t256_t256x128", 2, 112 + 32),  # gate/up t256w8 alone
        (4096, 14336, 256, "lf_fp8_w8a8_gated_mlp_t128_t128", 2, 224 + 32),
    ]:
        d, s = fp8.gated_mlp_geometry(h, i, m, _abi.ENTRY_W8A8_GATED_MLP)
        assert s == sym and d.grid == (512 + gx * bands, 1, 1) and d.block == (256, 1, 1), (s, d.grid)
        bm = 128 if "t128" in sym else 256
        cap = bands * bm
        sync = 256 + 128 * 3 * bands
        want = sync + fp8.act_quant_bytes(cap, h) + cap * i * 2 + fp8.act_quant_bytes(cap, i)
        assert lib.lunaflux_fp8_gated_mlp_workspace_bytes(_abi.ENTRY_W8A8_GATED_MLP, h, i, m) == want
    assert lib.lunaflux_fp8_gated_mlp_workspace_bytes(_abi.ENTRY_W8A8_GATED_MLP, 4000, 14336, 64) == -1


def test_block_scaled_geometry_and_workspace():
    """The _B128 entries. W8A16: profiles of 65..128 rows the LDS-tiled
    GEMM form (the _b128_m128_n{BN} symbols) by the per-channel rule (the
    most blocks up to 256, >= 8 k-tiles per slice) except that a tie goes to
    BN 128 instead of BN 64; the column-group form for every other profile
    (also <= 16 rows), the per-channel split raised so that a slice holds at
    most 128 k-tiles, the per-channel workspace formula. W8A8: 256 group-
    quantizer blocks then 128 x 128 tiles (64 h-columns for gate/up), 256
    threads; workspace = sync area + codes [cap, K] + scales [K/128][cap]
    (each part 256-aligned). GatedMlp: four steps on 128-row bands."""
    lib = _abi.lib()
    al = lambda v: -(-v // 256) * 256  # noqa: E731
    channel = {_abi.ENTRY_W8A16_DENSE_B128: _abi.ENTRY_W8A16_DENSE,
               _abi.ENTRY_W8A16_QKV_B128: _abi.ENTRY_W8A16_QKV,
               _abi.ENTRY_W8A16_GATE_UP_B128: _abi.ENTRY_W8A16_GATE_UP}
    for entry, op in [(_abi.ENTRY_W8A16_DENSE_B128, "dense"), (_abi.ENTRY_W8A16_QKV_B128, "qkv"),
                      (_abi.ENTRY_W8A16_GATE_UP_B128, "gate_up")]:
        # (BN, split) block-scaled / per-channel
        gate_up = op == "gate_up"
        for n, k, m, want_b, want_c in [
                (4096, 14336, 128, (128, 4) if gate_up else (128, 8), (64, 2) if gate_up else (64, 4)),
                (6144, 4096, 100, (128, 2) if gate_up else (128, 4), (64, 1) if gate_up else (64, 2)),
                (4096, 4096, 65, (128, 4) if gate_up else (64, 4), (64, 2) if gate_up else (64, 4)),
                (1024, 32768, 128, (128, 16) if gate_up else (128, 32), (64, 8) if gate_up else (64, 16))]:
            for e, sub, (bn, split) in ((entry, "_b128", want_b), (channel[entry], "", want_c)):
                d, sym = fp8.launch_geometry(e, n, k, m)
                blocks = n // (bn // 2 if gate_up else bn)
                assert sym == f"lf_fp8_w8a16_{op}{sub}_m128_n{bn}" and d.grid == (blocks * split, 1, 1), (sym, d)
                assert d.block == (512, 1, 1)
                want = 256 if split == 1 else al(split * blocks * 8 * 2 * (bn // 32) * 1024) + al(blocks * 4)
                assert fp8.w8a16_workspace_bytes(e, n, k, m) == want, (sym, split)
        # the Llama-3-8B shape-specialized forms at <= 32 rows: the per-channel
        # entry's geometry and workspace under the _b128 symbol
        for n, k, m, split in [(4096, 4096, 1, None), (4096, 4096, 32, None), (4096, 14336, 16, None),
                               (4096, 14336, 32, None), (14336, 4096, 8, None), (14336, 4096, 32, None),
                               (6144, 4096, 16, (4096, 1024)), (6144, 4096, 32, (4096, 1024))]:
            if (op == "qkv") != (split is not None) or (op == "gate_up") != (n == 14336):
                continue
            d, sym = fp8.launch_geometry(entry, n, k, m, split)
            d0, sym0 = fp8.launch_geometry(channel[entry], n, k, m, split)
            assert f"_k{k}" in sym0 and sym == sym0.replace(f"_{op}_", f"_{op}_b128_") and d == d0, (sym, sym0)
            ws0 = fp8.w8a16_workspace_bytes(channel[entry], n, k, m, split)
            # (QKV: sized without the split for every entry of that width)
            assert fp8.w8a16_workspace_bytes(entry, n, k, m) >= ws0
        for n, k, m, mt in [(4096, 2048, 1, 1), (6144, 2048, 32, 2), (14336, 4096, 64, 4),
                            (1024, 32768, 16, 1)]:
            d, sym = fp8.launch_geometry(entry, n, k, m)
            assert sym == f"lf_fp8_w8a16_{op}_b128_m{16 * mt}" and d.block == (256, 1, 1)
            groups = -(-(n // 16) // 4)
            assert d.grid[0] % groups == 0
            split = d.grid[0] // groups
            kt = k // 128
            assert 1 <= split <= kt and -(-kt // split) <= 128, (n, k, m, split)
            nw = 2 if op == "gate_up" else 1
            want = 256 if split == 1 else al(split * (n // 16) * nw * mt * 1024) + al(groups * 4)
            assert fp8.w8a16_workspace_bytes(entry, n, k, m) == want
    # 128-row blocks: N must be a multiple of 128, every QKV width too
    with pytest.raises(fp8.DeviceError):
        fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE_B128, 4096 + 64, 4096, 16)
    with pytest.raises(fp8.DeviceError):
        fp8.launch_geometry(_abi.ENTRY_W8A8_QKV_B128, 4096 + 2 * 1088, 4096, 256, qkv_split=(4096, 1088))
    # 256-row bands of 512 threads: the 256 x 256 form from 192 such tiles
    # on, where the width is a multiple of its tile, else 256 x 128 (128
    # columns; gate/up: 64 outputs); the 128 x 128 form (128-row bands, 256
    # threads) only for K >= 2^24. The workspace holds cap = bands x height
    # rows.
    for entry, op, n, k, m, t256 in [
            (_abi.ENTRY_W8A8_DENSE_B128, "dense", 4096, 14336, 2048, False),
            (_abi.ENTRY_W8A8_QKV_B128, "qkv", 6144, 4096, 300, False),
            (_abi.ENTRY_W8A8_GATE_UP_B128, "gate_up", 14336, 4096, 1, False),
            (_abi.ENTRY_W8A8_DENSE_B128, "dense", 4096, 4096, 3072, True),
            (_abi.ENTRY_W8A8_DENSE_B128, "dense", 4096, 14336, 3000, True),
            (_abi.ENTRY_W8A8_DENSE_B128, "dense", 4096, 4096, 2816, False),
            (_abi.ENTRY_W8A8_DENSE_B128, "dense", 4096 + 128, 4096, 8192, False),
            (_abi.ENTRY_W8A8_QKV_B128, "qkv", 6144, 4096, 2048, True),
            (_abi.ENTRY_W8A8_QKV_B128, "qkv", 6144, 4096, 1792, False),
            (_abi.ENTRY_W8A8_GATE_UP_B128, "gate_up", 14336, 4096, 300, True),
            (_abi.ENTRY_W8A8_GATE_UP_B128, "gate_up", 14336, 4096, 256, False),
            (_abi.ENTRY_W8A8_GATE_UP_B128, "gate_up", 1408, 4096, 8192, True)]:
        d, sym = fp8.launch_geometry(entry, n, k, m)
        bands = -(-m // 256)
        cols = 256 if t256 else 128
        gx = n // (cols // 2) if op == "gate_up" else n // cols
        assert sym == f"lf_fp8_w8a8_{op}_b128" + ("_t256" if t256 else "_t256x128"), (n, k, m, sym)
        assert d.grid == (256 + gx * bands, 1, 1) and d.block == (512, 1, 1)
        cap = 256 * bands
        want = 256 + 128 * bands + al(cap * k) + al((k // 128) * cap * 4)
        assert fp8.w8a8_workspace_bytes(entry, n, k, m) == want
    k = 1 << 24  # 32-bit activation offsets no longer fit: 128 x 128 tiles
    d, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_DENSE_B128, 256, k, 100)
    assert sym == "lf_fp8_w8a8_dense_b128" and d.grid == (256 + 2, 1, 1) and d.block == (256, 1, 1)
    assert fp8.w8a8_workspace_bytes(_abi.ENTRY_W8A8_DENSE_B128, 256, k, 100) == (
        256 + 128 + al(128 * k) + al((k // 128) * 128 * 4))
    d, sym = fp8.launch_geometry(_abi.ENTRY_W8A8_QKV_B128, 6144, 4096, 2048, qkv_split=(4096, 1024))
    assert sym == "lf_fp8_w8a8_qkv_b128_t256" and d.grid == (256 + 24 * 8, 1, 1)
    # block-scaled W8A8 GatedMlp: 128 x 128 tiles, or 256 x 256 ones (256-row
    # bands, 512 threads) where the gate/up launch takes them and the hidden
    # width is a multiple of 256 (no 256 x 128 form for it)
    e = _abi.ENTRY_W8A8_GATED_MLP_B128
    for h, i, m, bm in [(4096, 14336, 3072, 256), (4096, 14336, 2048, 256), (4096, 14336, 300, 256),
                        (4096, 14336, 256, 128), (4096, 2048, 3072, 256), (4096 + 128, 14336, 8192, 128),
                        (512, 1024, 100, 128)]:
        d, sym = fp8.gated_mlp_geometry(h, i, m, e)
        bands = -(-m // bm)
        cap = bm * bands
        assert sym == "lf_fp8_w8a8_gated_mlp_b128" + ("_t256" if bm == 256 else ""), (h, i, m, sym)
        assert d.grid == (512 + (i // (bm // 2) + h // bm) * bands, 1, 1) and d.block == (2 * bm, 1, 1)
        want = (256 + 128 * 3 * bands + al(cap * h) + al(h // 128 * cap * 4) + al(cap * i * 2)
                + al(cap * i) + al(i // 128 * cap * 4))
        assert lib.lunaflux_fp8_gated_mlp_workspace_bytes(e, h, i, m) == want
    assert lib.lunaflux_fp8_gated_mlp_workspace_bytes(e, 4096 + 64, 14336, 2048) == -1
    # W8A16 GatedMlp in one launch on block-scaled weights: at <= 32 rows the
    # per-channel one-launch forms' geometry and workspace under the _b128
    # symbols; at 65..128 rows the down part takes the block-scaled tie rule
    # (BN 128 x 8 slices where per-channel takes BN 64 x 4, both 256
    # blocks); none at 33..64 rows or at widths without a form
    e, e0 = _abi.ENTRY_W8A16_GATED_MLP_B128, _abi.ENTRY_W8A16_GATED_MLP
    for h, i, m in [(4096, 14336, 1), (4096, 14336, 32)]:
        d, sym = fp8.gated_mlp_geometry(h, i, m, e)
        d0, sym0 = fp8.gated_mlp_geometry(h, i, m, e0)
        assert sym == sym0.replace("gated_mlp_", "gated_mlp_b128_") and d == d0, (sym, sym0)
        assert (lib.lunaflux_fp8_gated_mlp_workspace_bytes(e, h, i, m)
                == lib.lunaflux_fp8_gated_mlp_workspace_bytes(e0, h, i, m))
    for h, i, m in [(4096, 14336, 128), (4096, 14336, 100)]:
        d, sym = fp8.gated_mlp_geometry(h, i, m, e)
        d0, sym0 = fp8.gated_mlp_geometry(h, i, m, e0)
        assert sym == "lf_fp8_w8a16_gated_mlp_b128_m128_n128_n128" and d.grid == (224 + 256, 1, 1), sym
        assert sym0 == "lf_fp8_w8a16_gated_mlp_m128_n128_n64" and d0.grid == (224 + 256, 1, 1), sym0
        for ee, bn, split in ((e, 128, 8), (e0, 64, 4)):
            blocks = h // bn
            down = split * blocks * 8 * 2 * (bn // 32) * 1024 + al(blocks * 4)
            assert lib.lunaflux_fp8_gated_mlp_workspace_bytes(ee, h, i, m) == 128 * i * 2 + down + 128 * split + 256
    assert fp8.gated_mlp_geometry(4096, 14336, 64, e) is None
    assert fp8.gated_mlp_geometry(2048, 5632, 32, e) is None
    assert fp8.gated_mlp_geometry(2048, 5632, 100, e) is None and fp8.gated_mlp_geometry(2048, 5632, 100, e0) is None


def test_block_scaled_admission_cpu():
    """Each entry admits only its own scale mode: LF_UNSUPPORTED across
    modes, LF_INVALID_ARGUMENT for an expert count on a dense entry."""
    rng = np.random.default_rng(3)
    qb, sb = synth.weight(rng, 256, 256, block=128)
    rb = fp8.pack_weight(qb, sb, fp8.BLOCK128)
    qc, sc = synth.weight(rng, 256, 256)
    rc = fp8.pack_weight(qc, sc)
    block_entries = (_abi.ENTRY_W8A16_DENSE_B128, _abi.ENTRY_W8A16_QKV_B128, _abi.ENTRY_W8A16_GATE_UP_B128,
                     _abi.ENTRY_W8A8_DENSE_B128, _abi.ENTRY_W8A8_QKV_B128, _abi.ENTRY_W8A8_GATE_UP_B128,
                     _abi.ENTRY_W8A8_GATED_MLP_B128)
    for entry in block_entries:
        fp8.admit_weight(entry, rb[:256], rb.size, 256, 256)
        with pytest.raises(fp8.DeviceError) as e:
            fp8.admit_weight(entry, rc[:256], rc.size, 256, 256)
        assert e.value.status == _abi.LF_UNSUPPORTED
    for entry in (_abi.ENTRY_W8A16_DENSE, _abi.ENTRY_W8A8_GATE_UP_AQ, _abi.ENTRY_W8A8_GATED_MLP):
        with pytest.raises(fp8.DeviceError) as e:
            fp8.admit_weight(entry, rb[:256], rb.size, 256, 256)
        assert e.value.status == _abi.LF_UNSUPPORTED
    fp8.admit_weight(_abi.ENTRY_GROUPED, rb[:256], rb.size, 256, 256)


def test_w8a16_gated_mlp_geometry():
    """One-launch W8A16 GatedMlp: the column-group entries at the Llama-3-8B
    widths for <= 16 / <= 32 rows; for 65..128 rows the LDS-tiled GEMMs
    (gate/up n128 unsplit, then the down launch's own tile and split) at any
    widths where gate/up takes n128 unsplit; none for 33..64 rows."""
    lib = _abi.lib()
    e = _abi.ENTRY_W8A16_GATED_MLP
    d, s = fp8.gated_mlp_geometry(4096, 14336, 32)
    assert s == "lf_fp8_w8a16_gated_mlp_h4096_i14336_m32" and d.grid == (224 + 256, 1, 1)
    d, s = fp8.gated_mlp_geometry(4096, 14336, 128)
    dn_dims, dn_sym = fp8.launch_geometry(_abi.ENTRY_W8A16_DENSE, 4096, 14336, 128)
    assert dn_sym == "lf_fp8_w8a16_dense_m128_n64"
    assert s == "lf_fp8_w8a16_gated_mlp_m128_n128_n64" and d.grid == (224 + dn_dims.grid[0], 1, 1)
    assert d.block == (512, 1, 1)
    ws = lib.lunaflux_fp8_gated_mlp_workspace_bytes(e, 4096, 14336, 128)
    split = dn_dims.grid[0] // (4096 // 64)
    assert ws == (128 * 14336 * 2 + fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_DENSE, 4096, 14336, 128)
                  + 128 * split + 256)       # one 128-byte line per slice counter, done, error
    assert (lib.lunaflux_fp8_gated_mlp_workspace_bytes(e, 4096, 14336, 32)
            == 32 * 14336 * 2 + fp8.w8a16_workspace_bytes(_abi.ENTRY_W8A16_DENSE, 4096, 14336, 32) + 768)
    assert fp8.gated_mlp_geometry(4096, 14336, 64) is None
    assert fp8.gated_mlp_geometry(1024, 2048, 128) is None   # gate/up would split K
    assert lib.lunaflux_fp8_gated_mlp_workspace_bytes(e, 4096, 14336, 64) == -1


class _FakeWorkspace:
    """The two calls BoundOperation.check makes on its workspace."""

    def __init__(self, nbytes):
        self.data = np.zeros(nbytes, np.uint8)
        self.byte_count = nbytes

    def read(self, dtype, shape, offset=0):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return self.data[offset:offset + n].view(dtype).reshape(shape).copy()

    def copy_from_host(self, data, offset=0):
        raw = np.ascontiguousarray(data).view(np.uint8).ravel()
        self.data[offset:offset + raw.size] = raw


def test_bound_operation_error_word():
    """A set error word (a counted wait ran out) raises LF_DRIVER_FAILURE and
    zero-fills the workspace, which puts its counters back at rest; a clear
    word passes; an operation without counted waits never reads."""
    ws = _FakeWorkspace(1024)
    op = fp8.BoundOperation([], workspace=ws, error_offset=0)
    op.check()
    ws.data[:4] = np.array([1], np.int32).view(np.uint8)
    ws.data[200] = 7                       # a counter left mid-count
    with pytest.raises(fp8.DeviceError) as err:
        op.check()
    assert err.value.status == _abi.LF_DRIVER_FAILURE
    assert not ws.data.any()
    op.check()
    ws2 = _FakeWorkspace(512)
    ws2.data[512 - _abi.LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END] = 1
    with pytest.raises(fp8.DeviceError):
        fp8.BoundOperation([], workspace=ws2, error_offset=512 - _abi.LF_FP8_GATED_MLP_ERROR_OFFSET_FROM_END).check()
    fp8.BoundOperation([], workspace=None).check()
    chain = fp8._Chain([], parts=[fp8.BoundOperation([], workspace=ws, error_offset=0), op])
    ws.data[:4] = np.array([1], np.int32).view(np.uint8)
    with pytest.raises(fp8.DeviceError):
        chain.check()


def test_closed_and_invalid_handles_without_gpu():
    lib = _abi.lib()
    status = ctypes.c_int32(0)
    ctx = lib.lunaflux_hip_context_create(0, ctypes.byref(status))
    if status.value == _abi.LF_OK:
        pytest.skip("a GPU is present")
    assert status.value in (_abi.LF_UNAVAILABLE, _abi.LF_INVALID_ARGUMENT)
    assert lib.lunaflux_hip_context_close(ctx) == _abi.LF_OK  # already closed
    s = lib.lunaflux_hip_stream_create(ctx, ctypes.byref(status))
    assert status.value == _abi.LF_CLOSED
    lib.lunaflux_hip_release(s)
    lib.lunaflux_hip_release(ctx)
    blas = lib.lunaflux_hip_blas_create(None, ctypes.byref(status))
    assert status.value == _abi.LF_UNSUPPORTED
    lib.lunaflux_hip_release(blas)
    assert lib.lunaflux_hip_bf16_gemm_plan_run(None, None, 0, None, 0, None, 0, None, 0, None) == _abi.LF_UNSUPPORTED


def test_numpy_quantizer_matches_oracle():
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 2 ** 32, 500_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    raw = raw[np.isfinite(raw)]
    np.testing.assert_array_equal(synth.e4m3_encode(raw), o.e4m3_encode(raw))
    np.testing.assert_array_equal(synth.bf16_bits(raw), o.bf16_round(raw))
    w = (rng.standard_normal((96, 512)) * 0.02).astype(np.float32)
    w[7] = 0
    for group in (None, 128):
        q1, s1 = synth.quantize_rows(w, group)
        q2, s2 = o.quantize_rows(w, group)
        np.testing.assert_array_equal(q1, q2)
        np.testing.assert_array_equal(s1, s2)
    wb = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    q1, s1 = synth.quantize_blocks(wb)
    q2, s2 = o.quantize_blocks(wb)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)


def test_golden_config1_reproduces_from_seed():
    g = np.load(os.path.join(ROOT, "tests", "golden", "config1.npz"))
    rng = np.random.default_rng(int(g["seed"]))
    x = synth.bf16_bits(rng.standard_normal((4, 512), dtype=np.float32))
    w = (rng.standard_normal((1536, 512), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    q, s = synth.quantize_rows(w)
    np.testing.assert_array_equal(x, g["x"])
    np.testing.assert_array_equal(q, g["q"])
    np.testing.assert_array_equal(s, g["s"])
    y = o.dense_projection(o.bf16_decode(x), o.dequantize(q, s))
    np.testing.assert_array_equal(y, g["y32"])


def test_moe_descriptor_layout_and_geometry():
    from lunaflux_amd import moe
    d = moe.moe_descriptor(8, 2, 0, 4096, 14336, 0)
    raw = d.as_bytes()
    assert raw.size == 32 and bytes(raw[:4]) == b"LMOE"
    lay = moe.workspace_layout(d, 1024)
    # (the workspace adds the down launch's counter area after the arrays)
    assert lay["end"] == moe.sync_offset(d, 1024) < moe.workspace_bytes(d, 1024)
    a = 1024 * 2
    assert lay["topk_w"] == a * 4 and lay["y"] + a * 4096 * 4 == lay["end"]
    assert all(v % 256 == 0 for v in lay.values())
    assert lay["xq"] - lay["tiles"] == 256  # 128- and 256-row tile prefixes, 2 x 9 int32
    dims, sym = moe.launch_geometry(4, d, 1024)   # gate/up
    # >= 256 routed rows per expert on average: 256 x 256 tiles, 1-D grid over
    # (128 h-column block, 256-row tile of the tile bound), 8 waves
    assert sym == "lf_moe_gate_up_t256" and dims.grid == (14336 // 128 * (a // 256 + 8), 1, 1)
    assert dims.block == (512, 1, 1)
    dims, sym = moe.launch_geometry(6, d, 1024)   # down, the hidden quantizer inside
    assert sym == "lf_moe_down_t256_aq" and dims.grid == (256 + 4096 // 256 * (a // 256 + 8), 1, 1)
    dims, sym = moe.launch_geometry(5, d, 1024)   # so no hidden-quantizer launch
    assert sym == "" and dims.grid == (0, 0, 0)
    # its counter area: error word, done counter, one line per 256-row tile
    # of the profile, at the end of the arrays for max_tokens
    sync_at = moe.sync_offset(d, 1024)
    assert sync_at == moe.workspace_layout(d, 1024)["end"]
    assert moe.workspace_bytes(d, 1024) == sync_at + -(-(256 + 128 * (a // 256 + 8 + 1)) // 256) * 256
    assert moe.sync_offset(d, 512) is None      # 128-row tiles: no counted step
    assert moe.workspace_bytes(d, 512) == moe.workspace_layout(d, 512)["end"]
    # the 256-row forms take 32-bit activation offsets: assignments x max(H, I)
    # must stay below 2^32 (here from 149,797 tokens at k = 2, I = 14336)
    for t, t256 in ((149796, True), (149797, False)):
        name = moe.launch_geometry(4, d, t)[1]
        assert (name == "lf_moe_gate_up_t256") == t256, (t, name)
    # fewer rows per expert: 128 x 128 tiles over (64 h-column block, 128-row tile)
    dims, sym = moe.launch_geometry(4, d, 512)
    assert sym == "lf_moe_gate_up" and dims.grid == (14336 // 64 * (512 * 2 // 128 + 8), 1, 1)
    dims, sym = moe.launch_geometry(2, d, 1024)   # sort: a block per 1024 assignments
    assert sym == "lf_moe_sort" and dims.grid == (2, 1, 1) and dims.block == (1024, 1, 1)
    dims, sym = moe.launch_geometry(8, d, 1024)   # sort counts: a block per 1024 assignments
    assert sym == "lf_moe_sort_count" and dims.grid == (2, 1, 1)
    dims, sym = moe.launch_geometry(1, d, 1024)   # route: a wave per token
    assert sym == "lf_moe_route" and dims.grid == (256, 1, 1) and dims.block == (256, 1, 1)
    # at most 1024 assignments: routing and the whole sort in one block, and
    # no sort launches (empty symbol, zero dims)
    for tokens in (512, 1):
        dims, sym = moe.launch_geometry(1, d, tokens)
        assert sym == "lf_moe_route_sort" and dims.grid == (1, 1, 1) and dims.block == (1024, 1, 1)
        for entry in (8, 2, 3):  # sort count, sort, token quantizer
            dims, sym = moe.launch_geometry(entry, d, tokens)
            assert sym == "" and dims.grid == (0, 0, 0) and dims.block == (0, 0, 0)
    assert moe.launch_geometry(1, d, 513)[1] == "lf_moe_route"
    assert moe.launch_geometry(2, d, 513)[1] == "lf_moe_sort"
    assert moe.launch_geometry(3, d, 513)[1] == "lf_moe_quant_tokens"
    d5 = moe.moe_descriptor(64, 6, 1, 2048, 1408, 128)
    # block scales averaging >= 256 rows per expert: 256 x 256 tiles too
    dims, sym = moe.launch_geometry(6, d5, 4096)  # down
    assert sym == "lf_moe_down_t256_b128" and dims.grid == (2048 // 256 * (4096 * 6 // 256 + 64), 1, 1)
    assert dims.block == (512, 1, 1)
    dims, sym = moe.launch_geometry(4, d5, 4096)  # gate/up, quantizing h in its epilogue
    assert sym == "lf_moe_gate_up_t256_b128_q" and dims.grid == (1408 // 128 * (4096 * 6 // 256 + 64), 1, 1)
    dims, sym = moe.launch_geometry(5, d5, 4096)  # so no hidden-quantizer launch
    assert sym == "" and dims.grid == (0, 0, 0) and dims.block == (0, 0, 0)
    assert moe.launch_geometry(5, d5, 2048)[1] == "lf_moe_quant_hidden"
    assert moe.launch_geometry(5, d5, 32)[1] == "lf_moe_quant_hidden"
    # fewer rows per expert, or K > 3072: 128 x 128 tiles
    dims, sym = moe.launch_geometry(6, d5, 2048)
    assert sym == "lf_moe_down_b128" and dims.grid == (2048 // 128 * (2048 * 6 // 128 + 64), 1, 1)
    d6 = moe.moe_descriptor(8, 2, 1, 4096, 1408, 128)
    assert moe.launch_geometry(4, d6, 4096)[1] == "lf_moe_gate_up_b128"
    # profiles of at most 32 tokens: the grouped GEMV form, a block per
    # (expert, 64 columns), either scale mode
    # (a fixed grid of at most 1024 blocks looping over the items)
    dims, sym = moe.launch_geometry(4, d5, 32)
    assert sym == "lf_moe_gate_up_gemv" and dims.grid == (1024, 1, 1) and dims.block == (256, 1, 1)
    dims, sym = moe.launch_geometry(6, d5, 32)
    assert sym == "lf_moe_down_gemv" and dims.grid == (1024, 1, 1)
    dims, sym = moe.launch_geometry(4, d, 16)
    assert sym == "lf_moe_gate_up_gemv" and dims.grid == (1024, 1, 1)   # 8 x 224 items, capped
    dims, sym = moe.launch_geometry(6, moe.moe_descriptor(8, 2, 0, 256, 384, 0), 1)
    assert sym == "lf_moe_down_gemv" and dims.grid == (2 * 256 // 64, 1, 1)   # at most k experts
    dims, sym = moe.launch_geometry(4, d5, 33)
    assert sym == "lf_moe_gate_up_b128"
    for bad in [(0, 1, 0, 256, 256, 0), (8, 9, 0, 256, 256, 0), (8, 2, 2, 256, 256, 0),
                (8, 2, 0, 200, 256, 0), (8, 2, 0, 256, 256, 64), (8, 2, 0, 8192, 256, 128)]:
        with pytest.raises(fp8.DeviceError):
            moe.moe_descriptor(*bad)


def test_rms_norm_quant_geometry():
    from lunaflux_amd import _abi, fp8
    from lunaflux_amd.device import DeviceError
    dims, sym = fp8.rms_norm_quant_geometry(1e-5, 4096, 130)
    assert sym == "lf_fp8_rms_norm_quant_rows_eps1em5"
    assert dims.grid == (33, 1, 1) and dims.block == (256, 1, 1)
    assert fp8.rms_norm_quant_geometry(1e-6, 8192, 4)[1] == "lf_fp8_rms_norm_quant_rows_eps1em6"
    with pytest.raises(DeviceError) as err:
        fp8.rms_norm_quant_geometry(1e-4, 4096, 16)
    assert err.value.status == _abi.LF_UNSUPPORTED
    for k, rows in ((8320, 16), (4000, 16), (4096, 0)):
        with pytest.raises(DeviceError) as err:
            fp8.rms_norm_quant_geometry(1e-5, k, rows)
        assert err.value.status == _abi.LF_INVALID_ARGUMENT
    with pytest.raises(DeviceError) as err:
        fp8.launch_geometry(_abi.ENTRY_RMS_NORM_QUANT_ROWS, 4096, 4096, 16)
    assert err.value.status == _abi.LF_INVALID_ARGUMENT


def test_pack_rejects_scale_and_code_counts_that_do_not_match_the_shape():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 256, (128, 256), dtype=np.uint8)
    # per channel wants N = 128 scales; block scales want (128/128)(256/128) = 2
    for scales, mode in [(np.ones(127, np.float32), fp8.PER_CHANNEL),
                         (np.ones(2, np.float32), fp8.PER_CHANNEL),
                         (np.ones(129, np.float32), fp8.PER_CHANNEL),
                         (np.ones(128, np.float32), fp8.BLOCK128),
                         (np.ones(1, np.float32), fp8.BLOCK128)]:
        with pytest.raises(fp8.DeviceError) as err:
            fp8.pack_weight(q, scales, mode)
        assert err.value.status == _abi.LF_INVALID_ARGUMENT
    # the C entry checks the code count too (the Python wrapper derives it
    # from q's shape, so call the library directly with a short count)
    size = fp8.weight_region_bytes(128, 256)
    region = np.empty(size, np.uint8)
    s = np.ones(128, np.float32)
    u8 = ctypes.POINTER(ctypes.c_uint8)
    f32 = ctypes.POINTER(ctypes.c_float)
    for q_bytes, count in [(q.size - 1, 128), (q.size, 127), (q.size + 16, 128)]:
        st = _abi.lib().lunaflux_fp8_pack_weight(
            fp8.PER_CHANNEL, 128, 256, 1, q.ctypes.data_as(u8), q_bytes, s.ctypes.data_as(f32),
            count, region.ctypes.data_as(u8), size)
        assert st == _abi.LF_INVALID_ARGUMENT
    assert fp8.scale_count(128, 256, 3, fp8.BLOCK128) == 6
    assert fp8.scale_count(128, 256, 3, fp8.PER_CHANNEL) == 384


DENSE_ENTRIES = (_abi.ENTRY_W8A16_DENSE, _abi.ENTRY_W8A16_QKV, _abi.ENTRY_W8A16_GATE_UP,
                 _abi.ENTRY_W8A8_DENSE, _abi.ENTRY_W8A8_QKV, _abi.ENTRY_W8A8_GATE_UP)


def test_admission_of_weight_regions():
    rng = np.random.default_rng(4)
    q = rng.integers(0, 0x7e, (256, 384), dtype=np.uint8)
    per = fp8.pack_weight(q, np.ones(256, np.float32))
    blk = fp8.pack_weight(q, np.ones(6, np.float32), fp8.BLOCK128)
    for entry in DENSE_ENTRIES:
        fp8.admit_weight(entry, per[:256], per.size, 256, 384)
        with pytest.raises(fp8.DeviceError) as err:
            fp8.admit_weight(entry, blk[:256], blk.size, 256, 384)
        assert err.value.status == _abi.LF_UNSUPPORTED
    # the grouped (MoE) entries read block scales
    fp8.admit_weight(_abi.ENTRY_GROUPED, blk[:256], blk.size, 256, 384)
    fp8.admit_weight(_abi.ENTRY_GROUPED, per[:256], per.size, 256, 384)
    experts = fp8.pack_weight(np.stack([q, q]), np.ones((2, 6), np.float32), fp8.BLOCK128)
    fp8.admit_weight(_abi.ENTRY_GROUPED, experts[:256], experts.size, 256, 384, 2)

    def rejected(entry, head, size, rows=256, cols=384, experts=1):
        with pytest.raises(fp8.DeviceError) as err:
            fp8.admit_weight(entry, head, size, rows, cols, experts)
        assert err.value.status == _abi.LF_INVALID_ARGUMENT

    d = _abi.ENTRY_W8A16_DENSE
    rejected(d, per[:256], per.size - 1)            # region smaller than the format's
    rejected(d, per[:256], per.size + 256)          # or larger
    rejected(d, per[:256], per.size, rows=128)      # shape the operation expects differs
    rejected(d, per[:256], per.size, cols=512)
    rejected(d, per[:128], per.size)                # header bytes missing
    rejected(_abi.ENTRY_ACT_QUANT_ROWS, per[:256], per.size)   # not a weight operand
    rejected(d, experts[:256], experts.size, experts=2)       # dense entries take one expert
    for field, value in [(0, 0x12345678), (1, 2), (2, 7), (3, 3), (4, 272), (5, 256), (6, 2)]:
        bad = per[:256].copy()
        bad[4 * field:4 * field + 4] = np.frombuffer(np.uint32(value).tobytes(), np.uint8)
        rejected(d, bad, per.size)
    for field in range(4):                          # tile/scale offsets and sizes
        bad = per[:256].copy()
        view = bad[32:64].view(np.uint64)
        view[field] += 256
        rejected(d, bad, per.size)


def test_block_scaled_weights_bind_their_own_entries():
    """A block-scaled region bound to a dense, QKV or gate/up operation binds
    the _B128 entry of the family (its admission passes); the per-token
    GEMM-only W8A8 entry over pre-quantized rows refuses it (LF_UNSUPPORTED)
    before anything is allocated or launched, so no device is needed."""
    from types import SimpleNamespace
    rng = np.random.default_rng(12)
    q = rng.integers(0, 0x7e, (256, 256), dtype=np.uint8)
    region = fp8.pack_weight(q, np.ones(4, np.float32), fp8.BLOCK128)
    w = fp8.Fp8Weight(SimpleNamespace(byte_count=region.size), 256, 256, 1, fp8.BLOCK128,
                      region[:256].copy())
    rt = fp8.ProjectionRuntime.__new__(fp8.ProjectionRuntime)
    rt._w8a16 = lambda entry, *a, **kw: ("w8a16", entry)
    rt._w8a8_one_launch = lambda entry, *a, **kw: ("w8a8", entry)
    counts = SimpleNamespace(byte_count=20, ptr=None)
    binds = {"dense": lambda f: rt.bind_dense(f, counts, None, w, None, 16),
             "qkv": lambda f: rt.bind_qkv(f, counts, None, w, w, w, None, 16),
             "gate_up": lambda f: rt.bind_gate_up(f, counts, None, w, w, None, 16)}
    for op, bind in binds.items():
        for family in fp8.FAMILIES:
            assert bind(family) == (family, fp8._BLOCK_ENTRIES[(family, op)])
    with pytest.raises(fp8.DeviceError) as err:
        fp8.ProjectionRuntime.bind_dense_quantized(None, None, None, w, None, 16)
    assert err.value.status == _abi.LF_UNSUPPORTED
