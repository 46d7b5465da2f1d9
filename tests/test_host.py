"""CPU checks of the package's host-side logic (no GPU): the layouts the
adapters hand to the kernels."""
from importlib import import_module

import pytest
import torch


def _cm(B, HK, T, D=128):
    """[B, HK, T, D] K/V in the sconv's channel-major layout: the view of a
    [B, HK*D, T] tensor (stride 1 along T, stride T along head_dim)."""
    x = torch.zeros((B, HK * D, T), dtype=torch.bfloat16)
    return x.transpose(1, 2).view(B, T, HK, D).transpose(1, 2)


@pytest.mark.parametrize("B,T", [(1, 8), (3, 200), (6, 1536), (2, 16)])
def test_kv_rows_reads_channel_major_in_place(B, T):
    """compat._kv_rows hands channel-major K/V with 16-byte aligned dim rows
    (T % 8 == 0) to the kernels as a view of the same memory: run stride =
    batch stride, token stride 1, dim stride T (what the prefill's
    channel-major source and the KV write read in place)."""
    compat = import_module("tm-opt_amd.compat")
    HK, D = 4, 128
    k = _cm(B, HK, T, D)
    r = compat._kv_rows(k)
    assert r.shape == (B, T, HK, D)
    assert r.data_ptr() == k.data_ptr()
    assert r.stride()[1:] == (1, D * T, T)
    assert r.stride(0) % 8 == 0 and (B == 1 or r.stride(0) == HK * D * T)
    assert torch.equal(r, k.transpose(1, 2))


@pytest.mark.parametrize("B,T", [(3, 77), (1, 5), (2, 100)])
def test_kv_rows_copies_unaligned_channel_major(B, T):
    """Channel-major rows whose dim stride is not a multiple of 8 (T % 8 !=
    0) are read by neither kernel: a token-major copy with the same
    values (the adapter makes it before it touches any cache)."""
    compat = import_module("tm-opt_amd.compat")
    g = torch.Generator().manual_seed(B * 1000 + T)
    HK, D = 2, 128
    x = torch.randn((B, HK * D, T), generator=g).to(torch.bfloat16)
    k = x.transpose(1, 2).view(B, T, HK, D).transpose(1, 2)
    r = compat._kv_rows(k)
    assert r.data_ptr() != k.data_ptr() and r.is_contiguous()
    assert torch.equal(r, k.transpose(1, 2))


def test_kv_rows_token_major_views():
    """Token-major K/V (a [B, HK, T, D] view of [B, T, HK, D] rows, or a
    contiguous [B, HK, T, D]) are read in place; a size-1 batch axis with an
    odd stride is fixed up without a copy."""
    compat = import_module("tm-opt_amd.compat")
    B, HK, T, D = 3, 4, 37, 128
    a = torch.zeros((B, T, HK, D), dtype=torch.bfloat16).transpose(1, 2)
    b = torch.zeros((B, HK, T, D), dtype=torch.bfloat16)
    for x in (a, b):
        r = compat._kv_rows(x)
        assert r.data_ptr() == x.data_ptr() and r.stride(3) == 1
    one = torch.zeros((HK * D * 8 + 4,), dtype=torch.bfloat16)[:HK * D * 8]
    one = one.as_strided((1, HK, 8, D), (3, D * 8, 1, 8))
    r = compat._kv_rows(one)
    assert r.data_ptr() == one.data_ptr() and r.stride(0) % 8 == 0


def test_c3_lengths_cover_the_window_edges():
    """Config 3's seeded lengths (the first draw of its generator, as the
    GPU parity and bench runs make them) include sequences shorter than the
    window, the longest ones, and window starts in the middle of a page, so
    the full-size C3 parity test meets every window geometry."""
    wl = import_module("tm-opt_amd.workloads")
    n = wl.decode_lens(3, 128, 2048, 32768).long()
    assert int(n.min()) < 4096 < int(n.max())
    assert int(n.max()) > 30000
    assert bool((((n - 4096) % 16 != 0) & (n > 4096)).any())


def test_ring_pool_detects_swapool_rows():
    """Rings that are rows of one SwaPool tensor (the engine's pooled
    RingKV views) are recognised, with each cache's pool row, so that their
    appends go out as one launch; separate rings, a shared row or a
    non-contiguous view are not."""
    compat = import_module("tm-opt_amd.compat")

    class Ring:
        def __init__(self, k, v):
            self.k, self.v, self.n = k, v, 0

    W, HK, D = 64, 2, 128
    pk = torch.zeros((5, W, HK, D), dtype=torch.bfloat16)
    pv = torch.zeros_like(pk)
    got = compat._ring_pool([Ring(pk[s], pv[s]) for s in (3, 0, 2)])
    assert got is not None
    kpool, vpool, slots, per = got
    assert slots == [3, 0, 2] and per == W // 16
    assert kpool.shape == (5 * W // 16, 16, HK, D)
    assert kpool.data_ptr() == pk.data_ptr() and vpool.data_ptr() == pv.data_ptr()
    # page j of row s is pool page s * per + j
    pk[2, 16:32] = 1
    assert bool((kpool[2 * per + 1] == 1).all()) and not bool(kpool[2 * per].any())
    sep = [Ring(torch.zeros((W, HK, D), dtype=torch.bfloat16),
                torch.zeros((W, HK, D), dtype=torch.bfloat16)) for _ in range(2)]
    assert compat._ring_pool(sep) is None
    assert compat._ring_pool([Ring(pk[1], pv[1]), Ring(pk[1], pv[1])]) is None
    assert compat._ring_pool([Ring(pk[1], pv[2])]) is None
    odd = torch.zeros((3, W, HK, 2 * D), dtype=torch.bfloat16)[..., :D]
    assert compat._ring_pool([Ring(odd[0], odd[1])]) is None


def test_uniform_cu_made_once_per_shape():
    """The fused adapter's run offsets (0, T, .., B*T) are made once per
    (B, T, device) and reused, as an int32 tensor of B + 1 entries."""
    compat = import_module("tm-opt_amd.compat")
    dev = torch.device("cpu")
    a = compat._uniform_cu(3, 5, dev)
    assert a.dtype == torch.int32 and a.tolist() == [0, 5, 10, 15]
    assert compat._uniform_cu(3, 5, dev) is a
    b = compat._uniform_cu(3, 6, dev)
    assert b is not a and b.tolist() == [0, 6, 12, 18]
    assert compat._uniform_cu(1, 7, dev).tolist() == [0, 7]


def _run_bench(*args, env_extra=None):
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, **(env_extra or {}))
    return subprocess.run([sys.executable, os.path.join(root, "bench.py"),
                           *args], capture_output=True, text=True, env=env,
                          timeout=120, cwd=root)


@pytest.mark.parametrize("args,env_extra", [
    (("--gpus", "2"), None),
    (("--gpus", "8", "--steps", "3"), None),
    ((), {"WORLD_SIZE": "2"}),
])
def test_bench_refuses_more_than_one_gpu(args, env_extra):
    """bench.py measures one GPU: --gpus above 1, or a launcher's
    WORLD_SIZE above 1, ends with status 2 and a message saying so, before
    any GPU is touched (and prints no JSON line)."""
    r = _run_bench(*args, env_extra=env_extra)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_bench_fails_loudly_without_a_gpu():
    """Without a visible GPU the bench exits non-zero instead of timing a
    fallback (this container has none; skipped where one is visible)."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    r = _run_bench("--steps", "1", "--warmup", "0")
    assert r.returncode == 1
    assert "no GPU" in r.stderr
    assert r.stdout.strip() == ""
