"""Host-side logic on the CPU: packed weight layouts (emulated in numpy and checked against
the oracle's dequantisation), the device fp32->e4m3fn conversion (compiled for the host and
compared with torch on every representable neighbourhood), launch plans, query blocks,
the caller-side Sequence contract and a StubRunner engine loop, and bench byte counts."""

import os
import shutil
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import qwen2_ref as ref

ROOT = Path(__file__).resolve().parent.parent


# ----------------------------------------------------------------------------- layouts
def emulate_gptq_repack_dequant(qweight: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """numpy restatement of the packed int4 layout + dequant8 -> W^T [K, N] fp16.

    packed word (tile nt, group kg, lane l, j): column 16*nt + l%16, k = 128*kg + 32*j +
    8*(l//16) + e; code e at bit 2e (e even) / 16 + 2(e-1) (e odd); dequant: the fp16 of
    ((w >> 4r) & 0x000F000F) | 0x64006400 minus 1032 times the group scale."""
    K8, N = qweight.shape
    K = K8 * 8
    W = np.zeros((K, N), dtype=np.float16)
    src = qweight.astype(np.int64) & 0xFFFFFFFF
    for nt in range(N // 16):
        for kg in range(K // 128):
            for lane in range(64):
                n = nt * 16 + lane % 16
                for j in range(4):
                    kb = kg * 128 + 32 * j + 8 * (lane // 16)
                    s_word = int(src[kb // 8, n])
                    word = 0
                    for e in range(8):
                        code = (s_word >> (4 * e)) & 0xF
                        bit = 16 + 2 * (e - 1) if e & 1 else 2 * e
                        word |= code << bit
                    s = np.float16(scales[kg, n])
                    for r in range(4):
                        t = ((word >> (4 * r)) & 0x000F000F) | 0x64006400
                        lo = np.array([t & 0xFFFF], dtype=np.uint16).view(np.float16)[0]
                        hi = np.array([t >> 16], dtype=np.uint16).view(np.float16)[0]
                        for e_, h in ((2 * r, lo), (2 * r + 1, hi)):
                            v = np.float16(np.float16(h - np.float16(1032)) * s)
                            W[kb + e_, n] = v
    return W


def test_packed_int4_layout_reproduces_reference_dequant():
    from omniserver_amd.synth import gptq_random
    K, N = 256, 32
    qw, sc = gptq_random(K, N, 5, "layout")
    W = emulate_gptq_repack_dequant(qw.numpy(), sc.numpy())
    assert np.array_equal(W.astype(np.float32), ref.gptq_dequant(qw, sc).numpy())


def test_packed_fp16_offset_formula():
    """Element (n, k) of the packed fp16 table (gather in norm.hip) sits at
    (((n//16)*(K//32) + k//32)*64 + n%16 + 16*((k%32)//8))*8 + k%8 = where f16_pack puts it."""
    N, K = 32, 64
    w = np.arange(N * K).reshape(N, K)
    packed = np.zeros(N * K, dtype=np.int64)
    for nt in range(N // 16):
        for ks in range(K // 32):
            for lane in range(64):
                n = nt * 16 + lane % 16
                k = ks * 32 + 8 * (lane // 16)
                base = ((nt * (K // 32) + ks) * 64 + lane) * 8
                packed[base:base + 8] = w[n, k:k + 8]
    for n in (0, 5, 17, 31):
        for k in (0, 7, 8, 31, 32, 63):
            off = (((n // 16) * (K // 32) + k // 32) * 64 + n % 16 + 16 * ((k % 32) // 8)) * 8 + k % 8
            assert packed[off] == w[n, k]


# ----------------------------------------------------------------------------- e4m3fn
E4M3_SRC = r"""
#include "common.h"
#include <cstdio>
#include <cstring>
int main(int argc, char** argv) {
  FILE* fi = fopen(argv[1], "rb"); FILE* fo = fopen(argv[2], "wb");
  float f;
  while (fread(&f, 4, 1, fi) == 1) { unsigned char c = f32_to_e4m3fn(f); fwrite(&c, 1, 1, fo); }
  fclose(fi); fclose(fo); return 0;
}
"""


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_device_e4m3_conversion_matches_torch():
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    with tempfile.TemporaryDirectory() as d:
        src = Path(d) / "e4m3.cpp"
        src.write_text(E4M3_SRC)
        exe = Path(d) / "e4m3"
        r = subprocess.run([hipcc, "--offload-arch=gfx950", "-O1",
                            f"-I{ROOT / 'omniserver_amd/csrc'}", f"-I{ROOT / 'include'}", str(src),
                            "-o", str(exe)], capture_output=True, text=True)
        if r.returncode != 0:
            pytest.skip(f"host build failed: {r.stderr[:300]}")
        # every e4m3 value, the midpoints between neighbours (ties), and random values
        codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
        finite = codes[torch.isfinite(codes)].unique().sort().values
        mids = (finite[1:] + finite[:-1]) / 2
        g = torch.Generator().manual_seed(3)
        rnd = torch.randn(20000, generator=g) * torch.exp(torch.randn(20000, generator=g) * 3)
        vals = torch.cat([finite, mids, mids.nextafter(torch.tensor(1e9)),
                          mids.nextafter(torch.tensor(-1e9)), rnd.clamp(-460, 460),
                          torch.tensor([0.0, -0.0, 2.0 ** -10, 2.0 ** -9 * 0.5, 447.9, 448.0,
                                        463.9, -463.9])])
        fi, fo = Path(d) / "in.bin", Path(d) / "out.bin"
        fi.write_bytes(vals.numpy().astype(np.float32).tobytes())
        subprocess.run([str(exe), str(fi), str(fo)], check=True)
        got = np.frombuffer(fo.read_bytes(), dtype=np.uint8)
        want = vals.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]


# ----------------------------------------------------------------------------- plans / blocks
def test_query_blocks_cover_segments():
    from omniserver_amd.attention import query_blocks
    qb = query_blocks([5, 16, 17, 1], "cpu").tolist()
    assert qb == [[0, 5], [5, 16], [21, 16], [37, 1], [38, 1]]


def test_append_writer_metadata():
    """Chunked / mixed adapters (kv_prealloc.py:104-174): per-token slot, write position
    start+i and visible keys start+i+1; lengths = start+L after finish; bad segments raise."""
    from omniserver_amd.kv_cache import PreallocatedKVCache
    pool = PreallocatedKVCache(2, 4, 2, 64, 128, "cpu", n_heads=12)
    w = pool.mixed_cache([0, 1, 3], [1, 1, 5], [10, 3, 20])
    assert w.token_slot.tolist() == [0, 1, 3, 3, 3, 3, 3]
    assert w.token_pos.tolist() == [10, 3, 20, 21, 22, 23, 24]
    assert w.kv_len.tolist() == [11, 4, 21, 22, 23, 24, 25]
    assert w.seg == [1, 1, 5] and w.T == 7
    w.finish()
    assert pool.lengths.tolist() == [11, 4, 0, 25]
    c = pool.chunked_prefill_cache(3, 25)
    assert c.seg is None
    c.bind(6)
    assert c.token_pos.tolist() == list(range(25, 31)) and c.kv_len.tolist() == list(range(26, 32))
    with pytest.raises(ValueError):
        c.bind(7)                                   # built for 6 tokens
    with pytest.raises(ValueError):
        pool.mixed_cache([0], [5], [60])            # past max_len
    with pytest.raises(ValueError):
        pool.mixed_cache([1, 1], [1, 2], [0, 5])    # one slot twice
    with pytest.raises(ValueError):
        pool.mixed_cache([4], [1], [0])             # slot outside the pool
    packed = pool.packed_prefill_cache([0, 2], [3, 2])
    assert packed.token_pos.tolist() == [0, 1, 2, 0, 1] and packed.kv_len.tolist() == [1, 2, 3, 1, 2]


def _hf_fp16_state_dict(w, prefix="model."):
    """fp16 weight dict -> Hugging Face Qwen2-VL key names (q/k/v, gate/up split)."""
    nq, nkv = 12 * 128, 2 * 128
    sd = {prefix + "embed_tokens.weight": w["embed"], prefix + "norm.weight": w["norm"]}
    for i, l in enumerate(w["layers"]):
        lp = f"{prefix}layers.{i}."
        sd[lp + "input_layernorm.weight"] = l["in_norm"]
        sd[lp + "post_attention_layernorm.weight"] = l["post_norm"]
        for x, (a, b) in {"q": (0, nq), "k": (nq, nq + nkv), "v": (nq + nkv, nq + 2 * nkv)}.items():
            sd[lp + f"self_attn.{x}_proj.weight"] = l["qkv_w"][a:b].contiguous()
            sd[lp + f"self_attn.{x}_proj.bias"] = l["qkv_b"][a:b].contiguous()
        sd[lp + "self_attn.o_proj.weight"] = l["o_w"]
        I = l["gate_up_w"].shape[0] // 2
        sd[lp + "mlp.gate_proj.weight"] = l["gate_up_w"][:I].contiguous()
        sd[lp + "mlp.up_proj.weight"] = l["gate_up_w"][I:].contiguous()
        sd[lp + "mlp.down_proj.weight"] = l["down_w"]
    return sd


def test_checkpoint_ingest(tmp_path):
    """GPTQ and fp16 checkpoint ingest (marlin_linear.py:114-143, qwen2_llm.py:193-219): the
    AutoGPTQ / Hugging Face tensors written to safetensors come back as the same fused
    weight dicts; a missing tensor and an activation-order g_idx are rejected; qzeros and a
    trivial g_idx are accepted; both state-dict prefixes load."""
    from safetensors.torch import save_file
    from omniserver_amd import checkpoint, synth
    shape = synth.DecoderShape(vocab_size=512)
    w = synth.gptq_decoder(shape, seed=3, num_layers=2)
    sd = checkpoint.gptq_state_dict_from_decoder(w)
    K = 1536
    sd["model.layers.0.self_attn.q_proj.g_idx"] = torch.arange(K, dtype=torch.int32) // 128
    sd["model.layers.0.self_attn.q_proj.qzeros"] = torch.full((K // 128, 192), 0x77777777,
                                                              dtype=torch.int64).to(torch.int32)
    sd["visual.blocks.0.attn.qkv.weight"] = torch.zeros(4, 4, dtype=torch.float16)   # ignored
    save_file(sd, str(tmp_path / "model-00001-of-00001.safetensors"))
    w2 = checkpoint.gptq_decoder_from_state_dict(checkpoint.read_safetensors(str(tmp_path)))
    assert torch.equal(w2["embed"], w["embed"]) and torch.equal(w2["norm"], w["norm"])
    for a, b in zip(w["layers"], w2["layers"]):
        assert a.keys() == b.keys()
        for k in a:
            assert a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]), k
    bad = dict(sd)
    del bad["model.layers.1.mlp.down_proj.scales"]
    with pytest.raises(KeyError, match="down_proj.scales"):
        checkpoint.gptq_decoder_from_state_dict(bad)
    bad = dict(sd)
    bad["model.layers.0.self_attn.q_proj.g_idx"] = torch.randperm(K).to(torch.int32) // 128
    with pytest.raises(ValueError, match="desc_act"):
        checkpoint.gptq_decoder_from_state_dict(bad)
    f = synth.fp16_decoder(shape, seed=4, num_layers=2)
    for prefix in ("model.", "model.language_model."):
        f2 = checkpoint.fp16_decoder_from_state_dict(_hf_fp16_state_dict(f, prefix))
        assert torch.equal(f2["embed"], f["embed"])
        for a, b in zip(f["layers"], f2["layers"]):
            for k in a:
                assert torch.equal(a[k], b[k]), (prefix, k)


def test_decode_plan_and_split_counts():
    from omniserver_amd.kv_cache import MAX_ATTN_SPLITS, decode_plan
    for n in (1, 8, 16, 32, 64):
        for ctx in (64, 256, 1024, 4096):
            w, s = decode_plan(n, 2, ctx)
            assert w in (4, 8, 16) and 1 <= s <= MAX_ATTN_SPLITS
    assert decode_plan(32, 2, 4096) == (8, 4)
    from omniserver_amd._lib import lib
    assert lib().omni_gemm_slices(8960, 10) == 10
    assert lib().omni_gemm_slices(1536, 10) == 6


# ----------------------------------------------------------------------------- control plane
def test_sequence_finish_rules():
    from omniserver_amd.request import Request, SamplingParams, Sequence, Status
    s = Sequence(Request(prompt=[1, 2], sampling=SamplingParams(max_new_tokens=3,
                                                                stop_token_ids=[9])))
    s.prompt_token_ids = [1, 2]
    assert s.last_token_id() == 2
    s.append_token(5)
    assert not s.maybe_finish() and s.last_token_id() == 5
    s.append_token(9)
    assert s.maybe_finish() and s.status == Status.FINISHED
    t = Sequence(Request(prompt=[1], sampling=SamplingParams(max_new_tokens=2)))
    t.append_token(1)
    t.append_token(2)
    assert t.maybe_finish()


def test_stub_runner_engine_loop():
    """The reference's control-plane double (runners/base.py:60-91) driven like
    LLMEngine.step: prefill new sequences, decode running ones, retire finished."""
    from omniserver_amd.request import Request, SamplingParams, Sequence, Status
    from omniserver_amd.runner import StubRunner
    r = StubRunner("a b c")
    seqs = [Sequence(Request(prompt="x y z", sampling=SamplingParams(max_new_tokens=n)))
            for n in (1, 3, 5)]
    for s in seqs:
        r.tokenize(s)
    r.prefill(seqs)
    running = [s for s in seqs if s.status != Status.FINISHED]
    steps = 0
    while running:
        r.decode(running)
        running = [s for s in running if s.status != Status.FINISHED]
        steps += 1
    assert [s.output_token_ids for s in seqs] == [[0], [0, 1, 2], [0, 1, 2, 3, 4]]
    assert steps == 4
    assert r.detokenize(seqs[1], [0, 1, 2]) == "a b c "


def test_synth_is_deterministic():
    from omniserver_amd import synth
    a = synth.gptq_random(256, 32, 7, "x")
    b = synth.gptq_random(256, 32, 7, "x")
    c = synth.gptq_random(256, 32, 7, "y")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert not torch.equal(a[0], c[0])
    codes = ref.gptq_unpack(a[0])
    assert codes.min() >= 0 and codes.max() <= 15
    assert (a[1] > 0).all()


# ----------------------------------------------------------------------------- bench bytes
def test_bench_byte_accounting_matches_published_floor():
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    w4 = bench.weight_bytes("gptq")
    assert abs(w4 / 1e9 - 1.143) < 0.005
    w16 = bench.weight_bytes("fp16")
    assert abs(w16 / 1e9 - 3.087) < 0.005
    # config 3 averaged over its 128 steps (mean attended context ~2112): ~3.08 GB per step
    assert abs(bench.step_bytes("gptq", [2111] * 32) / 1e9 - 3.08) < 0.01
    # one fused attention launch: 32 x 2048 keys read + 32 new rows written, (K+V) x 2 heads
    # x 128 x 2 B, the qkv rows + bias in, the output out
    assert bench.attn_launch_bytes([2048] * 32) == (32 * 2049 * 1024 + 33 * 2048 * 2
                                                    + 32 * 12 * 128 * 2)


def test_vision_state_dict_prefixes():
    """The vision tower's tensors are taken under either checkpoint prefix (``visual.`` or
    the newer ``model.visual.``) and come back under ``visual.``; decoder keys are left out."""
    import torch
    from omniserver_amd.checkpoint import vision_state_dict
    t = torch.zeros(2)
    sd = {"visual.blocks.0.norm1.weight": t, "model.visual.merger.ln_q.weight": t,
          "model.layers.0.input_layernorm.weight": t, "model.embed_tokens.weight": t}
    out = vision_state_dict(sd)
    assert set(out) == {"visual.blocks.0.norm1.weight", "visual.merger.ln_q.weight"}
    assert vision_state_dict({"model.norm.weight": t}) == {}


# ----------------------------------------------------------------------------- cache protocol
def _cpu_pool(n_layers=2, rows=3, max_len=16):
    from omniserver_amd.kv_cache import PreallocatedKVCache
    return PreallocatedKVCache(n_layers, rows, 2, max_len, 8, "cpu", n_heads=12)


def test_cache_view_update_matches_reference_semantics():
    """_CacheView.update (kv_prealloc.py:263-270): the new key/value of each row goes to
    its write position (the length when the view was made), the valid window
    [:, :max(pos) + 1] comes back as [n, n_kv, L, hd], and lengths advance on the last
    layer only; a view_graph view (:90-92) writes at the caller's positions and never
    advances lengths."""
    pool = _cpu_pool()
    pool.lengths[:2] = torch.tensor([3, 5])
    view = pool.view(2)
    for layer in range(2):
        key = torch.full((2, 2, 1, 8), float(layer + 1), dtype=torch.float16)
        val = -key
        k, v = view.update(key, val, layer)
        assert k.shape == (2, 2, 6, 8) and v.shape == (2, 2, 6, 8)
        assert torch.equal(pool.k[layer][0, 3], key[0, :, 0]) and torch.equal(pool.k[layer][1, 5], key[1, :, 0])
        assert torch.equal(pool.v[layer][1, 5], val[1, :, 0])
        assert torch.equal(k[1, :, 5], key[1, :, 0])
        want = [3, 5] if layer == 0 else [4, 6]
        assert pool.lengths[:2].tolist() == want
    assert view.get_seq_length() == 5 and view.get_mask_sizes(None) == (6, 0)
    assert view.get_max_cache_shape() == 16

    wp = torch.tensor([7, 1], dtype=torch.int64)
    g = pool.view_graph(2, wp, None, None)
    k, _ = g.update(torch.ones(2, 2, 1, 8, dtype=torch.float16), torch.ones(2, 2, 1, 8,
                    dtype=torch.float16), 1)
    assert k.shape[2] == 16 and pool.lengths[:2].tolist() == [4, 6]
    assert pool.k[1][0, 7].eq(1).all() and pool.k[1][1, 1].eq(1).all()
    g.finish()
    assert pool.lengths[:2].tolist() == [4, 6]
    view.finish()
    assert pool.lengths[:2].tolist() == [5, 7]


def test_prefill_writers_update():
    """_PackedPrefillWriter.update / _PrefillWriter.update (kv_prealloc.py:205-229): each
    segment of the packed [1, n_kv, T, hd] keys lands in its slot; lengths on the last
    layer; the keys come back unchanged."""
    pool = _cpu_pool()
    w = pool.packed_prefill_cache([2, 0], [3, 4])
    k = torch.arange(7, dtype=torch.float16).view(1, 1, 7, 1).expand(1, 2, 7, 8).contiguous()
    for layer in range(2):
        rk, rv = w.update(k, -k, layer)
        assert rk is k
    assert pool.lengths.tolist() == [4, 0, 3]
    assert pool.k[1][2, :3, 0, 0].tolist() == [0, 1, 2]
    assert pool.k[1][0, :4, 1, 0].tolist() == [3, 4, 5, 6]
    assert pool.v[0][0, 3, 0, 0].item() == -6
    single = pool.prefill_cache(1)
    for layer in range(2):
        single.update(k[:, :, :5], k[:, :, :5], layer)
    assert pool.lengths.tolist() == [4, 5, 3] and pool.k[0][1, :5, 0, 0].tolist() == [0, 1, 2, 3, 4]


def test_decode_addnorm_eligibility():
    """The 5-launch decode chain is taken only for up to decode_addnorm_rows rows whose norms
    fit the fused forms (hidden % 512 == 0, rows x hidden / 8 <= 512 threads)."""
    from types import SimpleNamespace
    from omniserver_amd.qwen2_llm import Qwen2LLM
    m = SimpleNamespace(cfg=SimpleNamespace(hidden_size=1536), decode_addnorm_rows=2)
    ok = lambda n: Qwen2LLM._addnorm_ok(m, n)
    assert ok(1) and ok(2) and not ok(3) and not ok(0)
    m.cfg.hidden_size = 1280                 # not whole waves per row
    assert not ok(1)
    m.cfg.hidden_size = 3072                 # 384 threads a row: one row only
    assert ok(1) and not ok(2)
    m.cfg.hidden_size, m.decode_addnorm_rows = 1536, 0
    assert not ok(1)


def test_prefill_k_slices():
    """Prefill K slices of the tiled GEMM (tile_ksplit): fp16 linears fill one round of the
    256 CUs with slices of at least two 128-groups (the 2B decoder at 256 rows: qkv / o 6,
    down 10); GPTQ linears keep at most 8 slices of four groups; no split for the SiLU-fused
    projection, at most 64 rows, or where the tiles already fill half the CUs."""
    from types import SimpleNamespace
    from omniserver_amd.linear import F16Linear, GPTQLinear
    from omniserver_amd._lib import lib

    def ks(cls, N, K, M, silu=False):
        lin = SimpleNamespace(N=N, K=K, fuse_silu=silu, FILL_SLICES=cls.FILL_SLICES)
        return cls.tile_ksplit(lin, M)

    shapes = {"qkv": (2048, 1536), "o": (1536, 1536), "down": (1536, 8960)}
    assert [ks(F16Linear, N, K, 256) for N, K in shapes.values()] == [6, 6, 10]
    assert [ks(GPTQLinear, N, K, 256) for N, K in shapes.values()] == [3, 3, 8]
    assert ks(F16Linear, 17920, 1536, 256, silu=True) == 1
    assert ks(F16Linear, 2048, 1536, 64) == 1
    for M in range(65, 1281, 37):
        for N, K in shapes.values():
            s = ks(F16Linear, N, K, M)
            tiles = -(-M // 128) * (N // 128)
            slices = lib().omni_gemm_slices(K, s)
            assert tiles * slices <= 256 or s == 1, (M, N, K, s)
            assert K // 128 // slices >= 2, (M, N, K, s)
