"""Selection parity at the headline and long-context lengths (T = 16384 and
65536, k = 2048): the selector's contract -- given identical fp32 scores, the
selected index sets are bit-exact with the reference selector
(gsa_ref.py:138-150, sorted ascending as gsa_opt.py:473-483,674-677 do) --
checked on the GPU's own scores.

The score kernel writes the full [1,T,T] fp32 matrix (1 GiB at 16384, 16 GiB
at 65536); on sampled rows (the trivial-row boundary t = k-2 .. k+1, the
middle, the last two rows -- at 65536 the last row has 65536 causal keys and
takes the fused kernel's 32-bit histogram variant -- and random rows) the
oracle's tie-aware selector runs on those rows copied to the host, and must
equal, bit for bit:
  * the standalone GPU selector over the whole matrix (ascending indices, counts);
  * the fused indexer + select (bitmask, ascending indices, counts), on its
    normal path and on its exact fallback.
Every row (not only the sampled ones) of the fused selection is also compared
with the standalone selector's on the GPU.
"""

import numpy as np
import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import _abi
from oracle import gsa_oracle as orc

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _rows(T, k, n=72, seed=0):
    fixed = {0, 1, 7, k - 2, k - 1, k, k + 1, T // 2, T // 2 + 1, T - 2, T - 1}
    rng = np.random.default_rng(seed)
    extra = rng.choice(np.arange(k + 2, T - 2), size=n - len(fixed), replace=False)
    return sorted(fixed | {int(r) for r in extra})


def _projections(T, dev, seed):
    """The indexer's inputs as the layer makes them: x ~ N(0,1) [1,T,2048] bf16
    through bf16 weights N(0, 0.02), q/k/w strided views of one buffer."""
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(1, T, 2048, device=dev, generator=g).to(torch.bfloat16)
    W = (torch.randn(328, 2048, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    proj = torch.nn.functional.linear(x, W)
    del x
    return proj[..., :256].view(1, T, 4, 64), proj[..., 256:320], proj[..., 320:324]


def _bits_of(idx, cnt, T):
    """uint32 selection words [n, W] of ascending (idx, count) rows, on the host."""
    n = idx.shape[0]
    W = _abi.mask_words(T)
    out = np.zeros((n, W), np.uint32)
    for r in range(n):
        sel = idx[r, :int(cnt[r])].astype(np.int64)
        np.bitwise_or.at(out[r], sel >> 5, (np.uint32(1) << (sel & 31).astype(np.uint32)))
    return out


@pytest.mark.parametrize("T", [16384, 65536])
def test_selection_bitexact_vs_oracle_on_gpu_scores(dev, T):
    k = 2048
    _log(f"selection vs oracle on GPU scores T={T} k={k}")
    q, kk, w = _projections(T, dev, seed=T)
    bias = torch.zeros(4, device=dev)
    rows = _rows(T, k, seed=T)
    s = _abi.indexer_scores(q, kk, w, bias, 0.125)                  # [1,T,T] fp32
    ui, uc, _ = _abi.topk_select(s, k, _abi.ORDER_INDEX_ASC)         # standalone selector, every row
    sr = s[0, rows].cpu()                                            # the sampled rows, on the host
    del s
    torch.cuda.synchronize()
    oi, oc = orc.select_ascending(sr[None], k)                      # the oracle on the same scores
    oi, oc = oi[0], oc[0]
    _log(f"  {len(rows)} sampled rows; counts {int(oc.min())}..{int(oc.max())}")
    assert torch.equal(uc[0, rows].cpu(), oc)
    assert torch.equal(ui[0, rows].cpu(), oi)
    want_bits = _bits_of(oi.numpy(), oc.numpy(), T)
    for forced in (False, True):
        _log(f"  fused select forced_fallback={forced}")
        if forced:
            with _abi.forced_select_fallback():
                fb, fi, fc = _abi.indexer_select(q, kk, w, bias, 0.125, k)
        else:
            fb, fi, fc = _abi.indexer_select(q, kk, w, bias, 0.125, k)
        torch.cuda.synchronize()
        assert torch.equal(fc[0, rows].cpu(), oc)
        assert torch.equal(fi[0, rows].cpu(), oi)
        assert np.array_equal(fb[0, rows].cpu().numpy().view(np.uint32), want_bits)
        # every row: fused == standalone selector on the same scores
        assert torch.equal(fc, uc) and torch.equal(fi, ui)
        del fb, fi, fc
