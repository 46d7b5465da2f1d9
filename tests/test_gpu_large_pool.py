"""Page pools larger than 4 GiB: every kernel addresses pages with 64-bit
byte offsets.

A 300,000-page pool (4.9 GB for K, the same for V, at 4 KV heads x 128 dims,
16 tokens per page) with the sequence's pages at the top of the pool, so
its rows sit past 2^32 bytes: the paged KV write must land them there
bit-exact, and decode and paged prefill must read them back, against fp32
references computed from the rows themselves.
"""
import pytest
import torch

from helpers import assert_lse_close, assert_out_close

pytestmark = pytest.mark.gpu

NUM_PAGES = 300_000
HQ, HKV, D, PAGE = 32, 4, 128, 16


def _ref(q, k, v, scale, causal_from=None):
    """fp32 attention of q [R, HQ, D] over k / v [n, HKV, D]; row r sees keys
    0 .. causal_from + r (all keys when causal_from is None)."""
    rep = HQ // HKV
    kf, vf = k.float(), v.float()
    outs, lses = [], []
    for r in range(q.shape[0]):
        n = k.shape[0] if causal_from is None else causal_from + r + 1
        qv = q[r].float().view(HKV, rep, D)
        s = torch.einsum("grd,ngd->grn", qv, kf[:n]) * scale
        lses.append(torch.logsumexp(s, -1).reshape(HQ))
        outs.append(torch.einsum("grn,ngd->grd", torch.softmax(s, -1),
                                 vf[:n]).reshape(HQ, D))
    return torch.stack(outs), torch.stack(lses)


def test_pool_past_4gib(tm, dev):
    g = torch.Generator(device=dev).manual_seed(41)
    T = 2000
    n_pages = (T + PAGE - 1) // PAGE
    # the top n_pages pages of the pool, in shuffled order
    top = torch.arange(NUM_PAGES - n_pages, NUM_PAGES, dtype=torch.int32)
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(3))
    table = top[perm][None].contiguous().to(dev)
    assert int(table.min()) * PAGE * HKV * D * 2 > 2 ** 32
    k_pool = torch.zeros((NUM_PAGES, PAGE, HKV, D), dtype=torch.bfloat16,
                         device=dev)
    v_pool = torch.zeros_like(k_pool)
    k = torch.randn((T, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((T, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, T], dtype=torch.int32, device=dev)
    tm.kv_write_paged(k, v, table, torch.zeros(1, dtype=torch.int32,
                                                device=dev),
                      k_pool, v_pool, cu_seqlens=cu, max_seqlen=T)
    torch.cuda.synchronize()
    pages = table[0].long()
    assert torch.equal(k_pool[pages].reshape(-1, HKV, D)[:T], k)
    assert torch.equal(v_pool[pages].reshape(-1, HKV, D)[:T], v)

    scale = D ** -0.5
    # decode of the 2000-token context
    q = torch.randn((1, HQ, D), generator=g, device=dev).to(torch.bfloat16)
    out, lse = tm.decode_paged(q, k_pool, v_pool, table,
                               torch.tensor([T], dtype=torch.int32,
                                            device=dev), scale)
    torch.cuda.synchronize()
    ref_o, ref_l = _ref(q.cpu(), k.cpu(), v.cpu(), scale)
    assert_out_close(out.cpu(), ref_o, "decode, pool past 4 GiB")
    assert_lse_close(lse.cpu(), ref_l, "decode, pool past 4 GiB")

    # prefill of the last 64 tokens with every key read from the pages
    R = 64
    qp = torch.randn((R, HQ, D), generator=g, device=dev).to(torch.bfloat16)
    out, lse = tm.prefill_varlen(
        qp, None, None, torch.tensor([0, R], dtype=torch.int32, device=dev),
        scale, prior_lens=torch.tensor([T - R], dtype=torch.int32,
                                       device=dev),
        k_pool=k_pool, v_pool=v_pool, block_table=table, max_seqlen=R)
    torch.cuda.synchronize()
    ref_o, ref_l = _ref(qp.cpu(), k.cpu(), v.cpu(), scale,
                        causal_from=T - R)
    assert_out_close(out.cpu(), ref_o, "paged prefill, pool past 4 GiB")
    assert_lse_close(lse.cpu().T, ref_l, "paged prefill, pool past 4 GiB")
