"""omni_lmhead_argmax_noalloc (lm_head + greedy argmax with library-held candidate slots)
against the allocating pair omni_lmhead_candidates + omni_argmax_finalize (candidates in
caller buffers), through the C ABI: two calls in a row, the second with a smaller input,
ids / logits / next_ids / lengths bit-equal; shapes beyond the library's array rejected
before any launch."""

import pytest
import torch

pytestmark = pytest.mark.gpu

H = 1536


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def _case(gpu, M, V, seed):
    from omniserver_amd.linear import LMHeadArgmax
    g = torch.Generator().manual_seed(seed)
    E = (torch.randn(V, H, generator=g) * 0.02).half()
    h = torch.randn(M, H, generator=g).half()
    E[7] = E[3]                          # two equal columns: ties resolve to the lower index
    return LMHeadArgmax(E.to(gpu)), h.to(gpu)


def _noalloc(lm, h, M, V, logits, ids, nxt, lens):
    from omniserver_amd._lib import lib, ptr, stream
    return lib().omni_lmhead_argmax_noalloc(ptr(h), h.stride(0), ptr(lm.table_packed), M, V, H,
                                            ptr(logits), ptr(ids), ptr(nxt), ptr(lens), stream())


def test_noalloc_lmhead_argmax_matches_allocating_path(gpu):
    for M, V, seed in ((33, 151936, 1), (5, 32768, 2)):      # the second call is smaller
        say(f"no-alloc lm_head argmax M={M} V={V}")
        lm, h = _case(gpu, M, V, seed)
        ids_ref = torch.empty(M, dtype=torch.int64, device=gpu)
        logits_ref = torch.empty(M, V, dtype=torch.float16, device=gpu)
        lm.argmax_out(h, ids_ref, logits_ref)
        ids = torch.full((M,), -1, dtype=torch.int64, device=gpu)
        nxt = torch.full((M,), -1, dtype=torch.int64, device=gpu)
        lens = torch.arange(M, dtype=torch.int64, device=gpu) * 3
        logits = torch.empty(M, V, dtype=torch.float16, device=gpu)
        assert _noalloc(lm, h, M, V, logits, ids, nxt, lens) == 0
        torch.cuda.synchronize()
        assert torch.equal(ids.cpu(), ids_ref.cpu())
        assert torch.equal(logits.cpu(), logits_ref.cpu())
        assert torch.equal(nxt.cpu(), ids.cpu())
        assert torch.equal(lens.cpu(), torch.arange(M, dtype=torch.int64) * 3 + 1)
        assert torch.equal(ids.cpu(), logits.float().cpu().argmax(-1))     # first max
        # without the optional outputs
        ids2 = torch.full((M,), -1, dtype=torch.int64, device=gpu)
        assert _noalloc(lm, h, M, V, None, ids2, None, None) == 0
        torch.cuda.synchronize()
        assert torch.equal(ids2.cpu(), ids_ref.cpu())


def test_noalloc_lmhead_argmax_rejects_oversize(gpu):
    from omniserver_amd._lib import lib
    say("no-alloc lm_head argmax: sizes beyond the library's array")
    L = lib()
    fake = 16                          # never dereferenced: the size checks come first
    assert L.omni_lmhead_argmax_noalloc(fake, H, fake, 65, 32768, H, None, fake, None, None,
                                        None) == -2
    assert L.omni_lmhead_argmax_noalloc(fake, H, fake, 4, 32760, H, None, fake, None, None,
                                        None) == -2
    assert L.omni_lmhead_argmax_noalloc(fake, H, fake, 4, 32768, H, None, None, None, None,
                                        None) == -1
