"""The decode read-floor diagnostic reads exactly the context rows of K and V.

Its per-item XOR checksums are compared bit-exactly with numpy over the same
rows (the words of every context token's K and V slot rows, gathered through
the block table on the CPU)."""

import numpy as np
import pytest
import torch

from mini_llm_runtime_amd.kernels import paged_attention as kpa

pytestmark = pytest.mark.gpu


def _expected(kc, vc, tables, lens, bs, tokens_per_item, items):
    k = kc.view(torch.int32).numpy().reshape(kc.shape[0] * bs, -1)
    v = vc.view(torch.int32).numpy().reshape(vc.shape[0] * bs, -1)
    out = np.zeros((len(lens), items), dtype=np.uint32)
    for b, n in enumerate(lens):
        for t in range(n):
            blk = tables[b][t // bs]
            if not 0 <= blk < kc.shape[0]:
                continue
            row = blk * bs + t % bs
            w = np.bitwise_xor.reduce(k[row].view(np.uint32)) ^ np.bitwise_xor.reduce(
                v[row].view(np.uint32))
            out[b, t // tokens_per_item] ^= w
    return out


@pytest.mark.parametrize("bs,hkv,d,tpi", [(16, 2, 64, 320), (16, 4, 128, 64), (32, 1, 64, 96),
                                          (16, 3, 64, 48)])
def test_read_floor_checksums(device, bs, hkv, d, tpi):
    gen = torch.Generator().manual_seed(bs * 1000 + hkv * 10 + d)
    nb = 64
    kc = torch.randint(-2**15, 2**15, (nb, bs, hkv, d), generator=gen, dtype=torch.int32)
    kc = kc.to(torch.int16).view(torch.bfloat16)
    vc = torch.randint(-2**15, 2**15, (nb, bs, hkv, d), generator=gen, dtype=torch.int32)
    vc = vc.to(torch.int16).view(torch.bfloat16)
    lens = [1, bs, 5 * bs + 3, 11 * bs, 0]
    width = 12
    perm = torch.randperm(nb, generator=gen).tolist()
    tables = [perm[i * width:(i + 1) * width] for i in range(len(lens))]
    tables[3][4] = -1          # an out-of-range id inside the context reads nothing
    tables[2][3] = nb + 3
    bt = torch.tensor(tables)
    got = kpa.paged_kv_read_floor(kc.to(device), vc.to(device), bt.to(device),
                                  torch.tensor(lens).to(device), tokens_per_item=tpi)
    items = (width * bs + tpi - 1) // tpi
    assert got.numel() == len(lens) * items
    want = _expected(kc, vc, tables, lens, bs, tpi, items)
    assert np.array_equal(got.cpu().numpy().view(np.uint32).reshape(len(lens), items), want)


def test_read_floor_rejects_bad_sizes(device):
    kc = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16, device=device)
    bt = torch.zeros(1, 2, dtype=torch.long, device=device)
    ctx = torch.tensor([20], device=device)
    with pytest.raises(Exception, match="tokens_per_item"):
        kpa.paged_kv_read_floor(kc, kc, bt, ctx, tokens_per_item=24)
