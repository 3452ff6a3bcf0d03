"""HIP KV append / metadata packing / block zeroing: bit-exact against the oracle and against
the CPU path of the same cache classes."""
import math

import numpy as np
import pytest
import torch

import oracle
from src.cache.paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState
from src.kernels.hip_paged_attention import kv_append_hip, pack_metadata_hip, zero_blocks_hip

pytestmark = pytest.mark.gpu


def _np_pool(t: torch.Tensor) -> np.ndarray:
    return oracle._np(t.cpu())


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_append_batch_gpu_matches_cpu_and_oracle(device, pool_dtype):
    g = torch.Generator().manual_seed(11)
    B, H, Hd, bs = 6, 4, 64, 16
    pools = {d: LayerBlockPool(block_size=bs, initial_blocks=4, growth_factor=2.0, dtype=pool_dtype) for d in ("cpu", "gpu")}
    states = {d: [PagedKVCacheState(pool=pools[d]) for _ in range(B)] for d in ("cpu", "gpu")}
    ref_k = ref_v = None
    ref_lens = [0] * B
    for step, T in enumerate([40, 1, 17, 1, 33]):
        k = torch.randn(B, T, H, Hd, generator=g).transpose(1, 2)  # strided like the model's views
        v = torch.randn(B, T, H, Hd, generator=g).transpose(1, 2)
        cur = torch.tensor([T, T - 1, 0, T + 5, max(T - 7, 0), 1][:B])
        print(f"append step {step} T={T}", flush=True)
        out_cpu = BatchedPagedKVCache(states["cpu"], pools["cpu"]).append_batch(k, v, cur)
        out_gpu = BatchedPagedKVCache(states["gpu"], pools["gpu"]).append_batch(k.to(device), v.to(device), cur)
        assert out_gpu.dtype == torch.long and out_gpu.cpu().tolist() == out_cpu.tolist()
        assert [s.block_ids for s in states["gpu"]] == [s.block_ids for s in states["cpu"]]
        assert pools["gpu"].free_block_ids == pools["cpu"].free_block_ids
        gk, ck = _np_pool(pools["gpu"].k_blocks), _np_pool(pools["cpu"].k_blocks)
        assert np.array_equal(gk, ck)
        assert np.array_equal(_np_pool(pools["gpu"].v_blocks), _np_pool(pools["cpu"].v_blocks))
        # oracle append on its own copy of the pool
        app = [max(min(int(c), T), 0) for c in cur]
        prev = list(ref_lens)
        ref_lens = [p + a for p, a in zip(prev, app)]
        shape = tuple(pools["gpu"].k_blocks.shape)
        nk = np.zeros(shape, dtype=gk.dtype)
        nv = np.zeros(shape, dtype=gk.dtype)
        if ref_k is not None:
            nk[: ref_k.shape[0]] = ref_k
            nv[: ref_v.shape[0]] = ref_v
        oracle.append(k.contiguous(), v.contiguous(), nk, nv, [s.block_ids for s in states["gpu"]], prev, app)
        ref_k, ref_v = nk, nv
        assert np.array_equal(gk, ref_k)
        assert np.array_equal(_np_pool(pools["gpu"].v_blocks), ref_v)
        pt, sl = BatchedPagedKVCache(states["gpu"], pools["gpu"]).device_metadata(device)
        assert np.array_equal(pt.cpu().numpy(), oracle.page_table([s.block_ids for s in states["gpu"]]))
        assert sl.cpu().tolist() == ref_lens


def test_kv_append_slot_mapping_and_conversion(device):
    g = torch.Generator().manual_seed(12)
    B, H, T, Hd, bs, N = 3, 2, 5, 16, 4, 9
    k_new = torch.randn(B, H, T, Hd, generator=g)
    v_new = torch.randn(B, H, T, Hd, generator=g)
    slots = torch.tensor([0, 5, -1, 35, 17, 2, 3, 4, -7, 8, 30, 31, 1, 6, 7], dtype=torch.int32)
    for pool_dtype in (torch.float32, torch.bfloat16):
        kp = torch.zeros(N, H, bs, Hd, dtype=pool_dtype, device=device)
        vp = torch.zeros_like(kp)
        kv_append_hip(k_new.to(device), v_new.to(device), kp, vp, slots.to(device))
        ek = torch.zeros(N, H, bs, Hd, dtype=pool_dtype)
        ev = torch.zeros_like(ek)
        for row, s in enumerate(slots.tolist()):
            if s < 0:
                continue
            b, j = divmod(row, T)
            ek[s // bs, :, s % bs] = k_new[b, :, j].to(pool_dtype)
            ev[s // bs, :, s % bs] = v_new[b, :, j].to(pool_dtype)
        assert torch.equal(kp.cpu(), ek) and torch.equal(vp.cpu(), ev)


def test_pack_metadata_bitwise(device):
    rng = np.random.default_rng(13)
    B, T, bs = 7, 9, 16
    lists = [rng.permutation(500)[: rng.integers(0, 12)].tolist() for _ in range(B)]
    prev = [max(0, len(x) * bs - int(rng.integers(0, 40))) for x in lists]
    app = [int(min(T, max(0, len(x) * bs - p))) for x, p in zip(lists, prev)]
    ids, offs = oracle.csr(lists)
    max_pages = max(len(x) for x in lists)
    dev = lambda a: torch.from_numpy(np.asarray(a, dtype=np.int32)).to(device)
    pt, s32, s64, slots = pack_metadata_hip(dev(ids), dev(offs), dev(prev), dev(app), query_len=T, block_size=bs,
                                            max_pages=max_pages)
    assert np.array_equal(pt.cpu().numpy(), oracle.page_table(lists))
    assert s32.cpu().tolist() == [p + a for p, a in zip(prev, app)] == s64.cpu().tolist()
    want = np.full(B * T, -1, dtype=np.int32)
    for b in range(B):
        for j in range(app[b]):
            p = prev[b] + j
            want[b * T + j] = lists[b][p // bs] * bs + p % bs
    assert np.array_equal(slots.cpu().numpy(), want)


def test_zero_blocks_and_release(device):
    kp = torch.randn(10, 2, 16, 64, device=device)
    vp = torch.randn_like(kp)
    keep_k, keep_v = kp.clone(), vp.clone()
    ids = [3, 7, 0, 42, -1]
    zero_blocks_hip(kp, vp, torch.tensor(ids, dtype=torch.int32, device=device))
    for i in range(10):
        if i in ids:
            assert torch.count_nonzero(kp[i]).item() == 0 and torch.count_nonzero(vp[i]).item() == 0
        else:
            assert torch.equal(kp[i], keep_k[i]) and torch.equal(vp[i], keep_v[i])
    pool = LayerBlockPool(block_size=16, initial_blocks=4, growth_factor=2.0)
    st = PagedKVCacheState(pool=pool)
    st.append(torch.randn(1, 2, 40, 64, device=device), torch.randn(1, 2, 40, 64, device=device), length=40)
    held = list(st.block_ids)
    st.release()
    assert torch.count_nonzero(pool.k_blocks).item() == 0
    assert pool.free_block_ids[-len(held):] == held
