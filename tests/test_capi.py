"""The C-ABI library: loads without a GPU, exports exactly what include/omniserver_amd.h
declares, the ctypes table matches the header's parameter counts, and argument
validation rejects bad shapes before any HIP call (safe to exercise on the CPU)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "omniserver_amd.h"


def header_decls():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\bint\s+(omni_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        decls[m.group(1)] = params
    return decls


@pytest.fixture(scope="module")
def so():
    from omniserver_amd._lib import LIB_PATH
    if not LIB_PATH.exists():
        pytest.fail("HIP library not built: run python -m omniserver_amd.build")
    return ctypes.CDLL(str(LIB_PATH))


def test_header_declares_entry_points():
    decls = header_decls()
    assert len(decls) >= 20
    assert "omni_decode_attention" in decls and "omni_w4a16_gemm" in decls


def test_library_exports_every_declared_symbol(so):
    for name in header_decls():
        assert hasattr(so, name), f"{name} declared in the header but not exported"


def test_ctypes_table_matches_header():
    from omniserver_amd._lib import SIGNATURES
    decls = header_decls()
    assert set(SIGNATURES) == set(decls)
    for name, params in decls.items():
        assert len(SIGNATURES[name]) == len(params), name


def fake_ptr():
    return ctypes.c_void_p(16)   # never dereferenced: validation fails first


def test_bad_arguments_rejected_before_launch(so):
    from omniserver_amd._lib import lib
    L = lib()
    # unsupported hidden size / negative rows
    assert L.omni_rmsnorm(None, None, None, 4, 7, 1e-6, None) == -2
    assert L.omni_rmsnorm(None, None, None, -1, 1536, 1e-6, None) == -1
    # null pointers with real work
    assert L.omni_add_rmsnorm(None, None, None, None, None, 4, 1536, 1e-6, None) == -1
    # attention: bad waves / head_dim / splits
    assert L.omni_decode_attention(None, 1536, None, None, 1, 16, None, None, 0, 0, None, 1, 12,
                                   2, 128, 0.1, 3, 1, None, 0, None) == -1
    assert L.omni_decode_attention(None, 1536, None, None, 1, 16, None, None, 0, 0, None, 1, 12,
                                   2, 64, 0.1, 4, 1, None, 0, None) == -2
    assert L.omni_decode_attention(None, 1536, None, None, 1, 16, None, None, 0, 0, None, 1, 12,
                                   2, 128, 0.1, 4, 0, None, 0, None) == -1
    # 16 waves per workgroup are no longer built; a workspace below the split states' size
    assert L.omni_decode_attention(fake_ptr(), 1536, fake_ptr(), fake_ptr(), 2, 16, None,
                                   fake_ptr(), 0, 0, fake_ptr(), 1, 12, 2, 128, 0.1, 16, 1, None,
                                   0, None) == -1
    assert L.omni_decode_attention(fake_ptr(), 1536, fake_ptr(), fake_ptr(), 2, 16, None,
                                   fake_ptr(), 0, 0, fake_ptr(), 1, 12, 2, 128, 0.1, 8, 4,
                                   fake_ptr(), 1 * 2 * 4 * 6 * 132 - 1, None) == -1
    # rotary rows: negative count, missing tables; the fused attention without rows needs them
    assert L.omni_rope_rows(None, None, None, None, None, 64, 4, -1, None, None) == -1
    assert L.omni_rope_rows(None, fake_ptr(), None, None, None, 64, 4, 2, fake_ptr(), None) == -1
    assert L.omni_decode_attention_fused(fake_ptr(), 6, None, 1, None, None, 64, None, 16, 24,
                                         24, fake_ptr(), fake_ptr(), 4, 64, None, fake_ptr(),
                                         fake_ptr(), 2, 12, 2, 128, 0.1, 8, 4, fake_ptr(),
                                         2 * 2 * 4 * 6 * 132, 1, None, None) == -1
    assert L.omni_decode_attention_fused(fake_ptr(), 6, None, 1, None, None, 64, None, 16, 24,
                                         24, fake_ptr(), fake_ptr(), 4, 64, None, fake_ptr(),
                                         fake_ptr(), 2, 12, 2, 128, 0.1, 8, 4, fake_ptr(),
                                         2 * 2 * 4 * 6 * 132 - 1, 1, fake_ptr(), None) == -1
    # slot copy: row out of range, row width not whole 16-byte chunks, device length without
    # a lengths array
    assert L.omni_kv_copy_slot(fake_ptr(), 2, 4, 64, 256, 0, 4, 3, None, None) == -1
    assert L.omni_kv_copy_slot(fake_ptr(), 2, 4, 64, 250, 0, 1, 3, None, None) == -2
    assert L.omni_kv_copy_slot(fake_ptr(), 2, 4, 64, 256, 0, 1, -1, None, None) == -1
    # vision tower: LayerNorm width past 2048, rotary head_dim not a multiple of 16,
    # attention head_dim other than 80, tiled GEMM kx past K / residual without res
    assert L.omni_layernorm(fake_ptr(), 2056, fake_ptr(), fake_ptr(), 4, 2056, 1e-6, fake_ptr(),
                            2056, None) == -2
    assert L.omni_vision_rope(fake_ptr(), 3840, 4, 16, 72, fake_ptr(), fake_ptr(), None) == -2
    assert L.omni_vit_attention(fake_ptr(), 3840, 4, 16, 64, fake_ptr(), fake_ptr(), 1,
                                fake_ptr(), 1280, 0.1, None) == -2
    assert L.omni_f16_gemm_tiled(fake_ptr(), 1280, 1288, fake_ptr(), None, None, 0, fake_ptr(),
                                 1280, 4, 1280, 1280, 0, None) == -1
    assert L.omni_f16_gemm_tiled(fake_ptr(), 1280, 1280, fake_ptr(), None, None, 0, fake_ptr(),
                                 1280, 4, 1280, 1280, 6, None) == -1
    # pipelined fp16 GEMM: K not a multiple of 64, slices below 4 K steps, split without
    # a workspace
    assert L.omni_f16_gemm_pipe(fake_ptr(), 1288, fake_ptr(), None, None, 0, fake_ptr(), 1280,
                                4, 1280, 1288, 0, 0, 1, None, None) == -2
    assert L.omni_f16_gemm_pipe(fake_ptr(), 1280, fake_ptr(), None, None, 0, fake_ptr(), 1280,
                                4, 1280, 1280, 0, 128, 8, None, None) == -2
    assert L.omni_f16_gemm_pipe(fake_ptr(), 1280, fake_ptr(), None, None, 0, fake_ptr(), 1280,
                                4, 1280, 1280, 0, 128, 2, None, None) == -1
    # GEMM: split-K partials past the skinny kernel's 64 rows, K not a multiple of 128,
    # split without partial epilogue; more rows with the STORE epilogue are the tiled GEMM
    # (here rejected for its null pointers, not its size)
    assert L.omni_w4a16_gemm(None, 1536, None, None, None, 1, None, 2048, None, 65, 2048, 1536,
                             2, 1, 2, None) == -2
    assert L.omni_w4a16_gemm(None, 1536, None, None, None, 1, None, 2048, None, 65, 2048, 1536,
                             0, 1, 2, None) == -1
    assert L.omni_w4a16_gemm(None, 1536, None, None, None, 1, None, 2048, None, 32, 2048, 1500,
                             0, 1, 2, None) == -2
    fake = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    assert L.omni_f16_gemm(fake, 1536, fake, None, fake, 2048, None, 32, 2048, 1536, 0, 4, 2,
                           None) == -1
    # rope: head_dim / sections
    assert L.omni_mrope_kv_write(None, 2048, None, None, None, None, None, 16, None, None, None,
                                 None, 1, 16, 1, 12, 2, 64, 16, 24, 24, None) == -2
    assert L.omni_mrope_kv_write(None, 2048, None, None, None, None, None, 16, None, None, None,
                                 None, 1, 16, 1, 12, 2, 128, 16, 24, 20, None) == -2
    # fp8: an output form past the three; per-tensor quantisation without its workspace or
    # with K not whole 8-element chunks; the workspace is one float per workgroup (<= 256)
    assert L.omni_fp8_gemm(fake_ptr(), fake_ptr(), fake_ptr(), fake_ptr(), None, fake_ptr(),
                           256, 8, 256, 256, 3, None) == -1
    # operands and bias staged with 16-byte loads: a misaligned pointer is rejected
    assert L.omni_fp8_gemm(ctypes.c_void_p(16 + 8), fake_ptr(), fake_ptr(), fake_ptr(), None,
                           fake_ptr(), 256, 8, 256, 256, 0, None) == -1
    assert L.omni_fp8_gemm(fake_ptr(), fake_ptr(), fake_ptr(), fake_ptr(), ctypes.c_void_p(16 + 2),
                           fake_ptr(), 256, 8, 256, 256, 0, None) == -1
    assert L.omni_fp8_quant_tensor(fake_ptr(), 256, fake_ptr(), fake_ptr(), None, 8, 256, 0,
                                   None) == -1
    assert L.omni_fp8_quant_tensor(fake_ptr(), 260, fake_ptr(), fake_ptr(), fake_ptr(), 8, 250,
                                   0, None) == -2
    assert L.omni_fp8_quant_weight_rows(None, 256, None, None, -1, 256, None) == -1
    assert [L.omni_fp8_quant_tensor_work(r) for r in (0, 1, 255, 256, 100000)] == [0, 1, 255,
                                                                                  256, 256]
    # prefill attention with the key tiles split between two wave groups: at most 6 query
    # heads per KV head (28 / 4 is rejected, 12 / 2 with no blocks is a no-op)
    assert L.omni_prefill_attention_gqa_halves(None, 28 * 128, None, None, 1, 16, None, None,
                                               None, 0, None, 28 * 128, 28, 4, 128, 0.1,
                                               None) == -2
    assert L.omni_prefill_attention_gqa_halves(None, 12 * 128, None, None, 1, 16, None, None,
                                               None, 0, None, 12 * 128, 12, 2, 128, 0.1,
                                               None) == 0
    # packed prefill GEMM plan: N not a multiple of 128, an unknown weight format
    assert L.omni_packed_gemm_pipe_plan(4096, 1500, 1536, 1, 0, 0, 0, 0, None, None, None) == -1
    assert L.omni_packed_gemm_pipe_plan(4096, 1536, 1536, 2, 0, 0, 0, 0, None, None, None) == -1
    # zero-size work is a no-op success
    assert L.omni_silu_mul(None, None, 0, 8960, None) == 0
    assert L.omni_gemm_slices(8960, 10) == 10 and L.omni_gemm_slices(1536, 7) == 6


def test_pipe_gemm_launch_choices(so):
    """The pipelined GEMM's host-side choice of K slices (no GPU needed: without a device the
    library assumes 256 CUs, the MI355X count).  The vision tower's shapes at 1024 patches:
    the qkv and fc1 tiles fill the grid (no split), proj / fc2 / the merger's linears leave
    CUs idle and are split; a full grid (M = 8192) is never split."""
    from omniserver_amd._lib import lib
    f = lib().omni_f16_gemm_pipe_splits
    assert f(1024, 3840, 1280, 0) == 1
    assert f(1024, 5120, 1280, 0) == 1
    assert f(1024, 1280, 1280, 0) == 2
    assert f(1024, 1280, 5120, 0) == 3
    assert f(256, 5120, 5120, 0) == 3
    assert f(256, 1536, 5120, 0) == 4
    assert f(8192, 1280, 5120, 0) == 1
    assert f(8192, 1280, 100, 0) == 1            # K % 128 != 0: never split


def test_packed_partial_plan(so):
    """The packed prefill GEMM's tiling for fp32 partial output with the K slices left to the
    plan (no GPU needed: 256 CUs assumed): config 5's down projection at M = 4096 on the
    persistent 256 x 192 tiles in 2 slices (128 tiles x 2 = one item per CU), a 2048-wide one
    on 256 x 256 tiles in 2 slices; the o projection (K = 1536) as well (its extra slice's
    traffic priced against the 128 x 192 tiles' cost); a caller's ksplit, int4 weights, or M
    not a multiple of 256 keep the pipelined tiles; the STORE plan is unchanged."""
    import ctypes
    from omniserver_amd._lib import lib
    L = lib()

    def plan(M, N, K, fmt, epi, ksplit=0):
        r, c, k = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
        assert L.omni_packed_gemm_pipe_plan(M, N, K, fmt, epi, 0, 0, ksplit, ctypes.byref(r),
                                            ctypes.byref(c), ctypes.byref(k)) == 0
        return r.value, c.value, k.value

    assert plan(4096, 1536, 8960, 1, 2) == (256, 192, 2)
    assert plan(4096, 2048, 8960, 1, 2) == (256, 256, 2)
    assert plan(4096, 1536, 1536, 1, 2) == (256, 192, 2)
    assert plan(4096, 1536, 8960, 1, 2, ksplit=1) == (128, 192, 1)
    assert plan(4096, 1536, 8960, 0, 2)[0:2] != (256, 192)
    assert plan(4000, 1536, 8960, 1, 2)[0] != 256
    assert plan(4096, 1536, 8960, 1, 0) == (128, 192, 1)
    assert plan(1024, 1536, 8960, 1, 2) == (128, 128, 2)


def test_packed_silu160_plan(so):
    """The SiLU-fused gate_up at 129-256 rows on packed fp16 weights takes 128 x 160 tiles
    (five gate|up pairs) where they fill the 256 CUs in one round (config 1's 256-token
    prompt: 224 tiles); 128 rows or fewer, more than 256, int4 weights, N not a multiple of
    160, too many tiles for one round or a forced tile height keep the other tiles."""
    import ctypes
    from omniserver_amd._lib import lib
    L = lib()

    def plan(M, N, K, fmt, epi, tile_rows=0):
        r, c, k = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
        assert L.omni_packed_gemm_pipe_plan(M, N, K, fmt, epi, 0, tile_rows, 0, ctypes.byref(r),
                                            ctypes.byref(c), ctypes.byref(k)) == 0
        return r.value, c.value, k.value

    assert plan(256, 17920, 1536, 1, 1) == (128, 160, 1)
    assert plan(129, 17920, 1536, 1, 1) == (128, 160, 1)
    assert plan(256, 1280, 512, 1, 1) == (128, 160, 1)
    assert plan(128, 17920, 1536, 1, 1)[1] == 128
    assert plan(257, 17920, 1536, 1, 1)[1] != 160
    assert plan(256, 17920, 1536, 0, 1)[1] != 160
    assert plan(256, 17920 + 128, 1536, 1, 1)[1] != 160
    assert plan(256, 25600 + 640, 1536, 1, 1)[1] != 160     # 2 x 164 tiles > 256 CUs
    assert plan(256, 17920, 1536, 1, 1, tile_rows=256) == (256, 128, 1)
    # the biased STORE / QGELU / GELU / RESID epilogues take them too where one round of
    # them covers more CUs than one round of 128-column tiles (the vision tower's fc1)
    assert plan(1024, 5120, 1280, 1, 4) == (128, 160, 1)
    assert plan(1024, 5120, 1280, 1, 0) == (128, 160, 1)
    assert plan(256, 17920, 1536, 1, 0) == (128, 160, 1)
    assert plan(1024, 1280, 5120, 1, 6)[1] != 160          # 64 tiles against 80
    assert plan(1024, 3840, 1280, 1, 0)[1] != 160          # 192 against 240
    assert plan(1024, 5120, 1280, 1, 2)[1] != 160          # partial sums keep their plan
    assert plan(4096, 5120, 1280, 1, 4)[1] != 160          # more than one round
