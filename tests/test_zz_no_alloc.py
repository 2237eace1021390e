"""gsa_indexer_select_noalloc (the select with no workspace argument, on the
library's static device array) against gsa_indexer_select: bit-identical
bitmasks, indices and counts on two calls in a row, the second smaller, so
that the second call runs on the array as the first left it."""

import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import _abi

pytestmark = pytest.mark.gpu


def _inputs(B, T, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    buf = torch.randn(B, T, 256 + 64 + 4 + 60, generator=g).to(dtype)
    bias = (torch.randn(4, generator=g) * 0.5).to(torch.float32)
    return buf, bias


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_select_matches_select_on_two_calls(dev, dtype):
    # (B, T, k): the first call covers 2 * 188 groups, the second fewer
    for B, T, k in [(2, 3000, 512), (1, 700, 64)]:
        print(f"noalloc select dtype={dtype} B={B} T={T} k={k}", flush=True)
        buf, bias = _inputs(B, T, dtype, seed=T)
        bd = buf.to(dev)
        q, kk, w = bd[..., :256].view(B, T, 4, 64), bd[..., 256:320], bd[..., 320:324]
        b32 = bias.to(dev)
        ref_bits, ref_idx, ref_cnt = _abi.indexer_select(q, kk, w, b32, 0.125, k)
        W = _abi.mask_words(T)
        bits = torch.full((B, T, W), -1, device=dev, dtype=torch.int32)
        idx = torch.full((B, T, k), -1, device=dev, dtype=torch.int32)
        cnt = torch.full((B, T), -1, device=dev, dtype=torch.int32)
        _abi.indexer_select_noalloc(q, kk, w, b32, 0.125, k, bits, idx, cnt)
        torch.cuda.synchronize()
        assert torch.equal(bits, ref_bits)
        assert torch.equal(idx, ref_idx)
        assert torch.equal(cnt, ref_cnt)
        # the selection itself: row t keeps min(t+1, k) keys
        pop = torch.tensor([bin(v & 0xffffffff).count("1") for v in bits[0, -1].tolist()]).sum().item()
        assert pop == min(T, k)


def test_noalloc_select_rejects_sizes_past_its_scratch(dev):
    # B=8193 at T=16: 8193 16-row groups, one more than the static array
    # holds; rejected on the host before anything is enqueued
    buf, bias = _inputs(1, 32, torch.bfloat16, seed=1)
    bd = buf.to(dev)
    q, kk, w = bd[..., :256].view(1, 32, 4, 64), bd[..., 256:320], bd[..., 320:324]
    bits = torch.zeros(1, 32, _abi.mask_words(32), device=dev, dtype=torch.int32)
    lib = _abi.load()
    st = lib.gsa_indexer_select_noalloc(q.data_ptr(), 0, 384, kk.data_ptr(), 0, 384, w.data_ptr(), 0, 384,
                                        bias.to(dev).data_ptr(), 0.125, 8193, 16, 4, 64, 8, _abi.DTYPE_BF16,
                                        bits.data_ptr(), 32, 2, None, None, None)
    assert st == 7


def test_noalloc_wrapper_checks_outputs_before_any_launch(dev):
    """The Python binding refuses outputs the kernels would overrun (idx/cnt of
    the wrong shape or dtype, bits of a narrower dtype) and inputs that
    gsa_indexer_select's binding refuses, before the library is called."""
    B, T, k = 1, 100, 16
    buf, bias = _inputs(B, T, torch.bfloat16, seed=3)
    bd = buf.to(dev)
    q, kk, w = bd[..., :256].view(B, T, 4, 64), bd[..., 256:320], bd[..., 320:324]
    b32 = bias.to(dev)
    W = _abi.mask_words(T)
    bits = torch.zeros(B, T, W, device=dev, dtype=torch.int32)
    idx = torch.zeros(B, T, k, device=dev, dtype=torch.int32)
    cnt = torch.zeros(B, T, device=dev, dtype=torch.int32)
    bad = [
        dict(idx=torch.zeros(B, T, k - 1, device=dev, dtype=torch.int32)),       # undersized idx
        dict(cnt=torch.zeros(B, T - 1, device=dev, dtype=torch.int32)),          # undersized cnt
        dict(idx=torch.zeros(B, T, k, device=dev, dtype=torch.int64)),           # idx dtype
        dict(bits=torch.zeros(B, T, W, device=dev, dtype=torch.int16)),          # narrower bits
        dict(w=bd[..., 320:323]),                                                # w [B,T,3]
        dict(b32=b32.to(torch.bfloat16)),                                        # bias dtype
        dict(kk=bd[..., 256:320].float()),                                       # mixed dtypes
    ]
    for over in bad:
        a = dict(q=q, kk=kk, w=w, b32=b32, bits=bits, idx=idx, cnt=cnt)
        a.update(over)
        with pytest.raises(ValueError):
            _abi.indexer_select_noalloc(a["q"], a["kk"], a["w"], a["b32"], 0.125, k, a["bits"], a["idx"], a["cnt"])
    _abi.indexer_select_noalloc(q, kk, w, b32, 0.125, k, bits, idx, cnt)
    torch.cuda.synchronize()
    assert int(cnt[0, -1]) == k
