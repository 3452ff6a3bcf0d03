"""HIP KV append / metadata packing / block zeroing: bit-exact against the oracle and against
the CPU path of the same cache classes."""
import math
import random

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


def test_pack_metadata_mirror_matches_csr_pack(device):
    """pa_pack_metadata_mirror over a random sequence of steps (appends, releases, hand edits, row
    take-over), with the descriptor in pinned host memory the kernel reads directly, against
    pa_pack_metadata from each step's full CSR lists: page tables, lengths and slots bit-exact, the
    staged words copied exactly, and the device mirror equal to the host shadow after every step."""
    from src.kernels.hip_paged_attention import pack_metadata_mirror_hip
    from src.kernels.staging import MappedHostWords
    from src.model.graph_decode import _step_metadata_py

    rng = random.Random(17)
    R, W, bs, T, Bmax = 6, 24, 16, 5, 4
    mirror = torch.full((R, W), -1, dtype=torch.int32, device=device)
    shadow, slen = np.full((R, W), -1, np.int32), np.zeros(R, np.int32)
    stage_words = 3 * Bmax
    # descriptor: [stage | mrow | first | num pages | prev | app | update ids, W per request]
    o_cur, o_sel, o_mrow = 0, Bmax, 2 * Bmax
    o_first, o_npages = 3 * Bmax, 4 * Bmax
    o_prev, o_app, o_upd = 5 * Bmax, 6 * Bmax, 7 * Bmax
    desc = MappedHostWords(o_upd + Bmax * W, device)
    addrs = {"mirror_row": desc.device_addr(o_mrow), "first_page": desc.device_addr(o_first),
             "num_pages": desc.device_addr(o_npages), "update_ids": desc.device_addr(o_upd), "update_stride": W,
             "prev_lens": desc.device_addr(o_prev), "append_lens": desc.device_addr(o_app),
             "stage_src": desc.device_addr(0)}
    stage = torch.zeros(stage_words, dtype=torch.int32, device=device)
    lists = {r: [] for r in range(R)}
    dev = lambda a: torch.from_numpy(np.asarray(a, dtype=np.int32)).to(device)
    for step in range(60):
        B = rng.randint(1, Bmax)
        rows = rng.sample(range(R), B)
        for r in rows:
            op = rng.random()
            if op < 0.7:
                lists[r] = (lists[r] + [rng.randrange(4000) for _ in range(rng.randint(0, 2))])[:W]
            elif op < 0.8:
                lists[r] = []
            elif op < 0.9 and lists[r]:
                lists[r][rng.randrange(len(lists[r]))] = rng.randrange(4000)
            else:
                slen[r] = 0  # taken over: resent whole
        states = [PagedKVCacheState(pool=None, block_ids=list(lists[r])) for r in rows]
        prev = [max(0, len(lists[r]) * bs - rng.randint(0, 20)) for r in rows]
        app = [min(T, max(0, len(lists[r]) * bs - p)) for r, p in zip(rows, prev)]
        cur = [rng.randint(0, 9) for _ in rows]
        sel = [rng.randint(0, 4) for _ in rows]
        desc.wait()
        desc.words[:] = -99
        lay = (o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, W)
        _step_metadata_py(states, rows, prev, app, cur, sel, shadow, slen, desc.words, lay)
        # stage region for this B: [cur B | sel B] packed at the front, as a graph step lays it out
        desc.words[0:B] = cur
        desc.words[B:2 * B] = sel
        max_pages = max(len(lists[r]) for r in rows) + 1
        print(f"mirror pack step {step}: B={B} rows={rows} max_pages={max_pages}", flush=True)
        pt, s32, s64, slots = pack_metadata_mirror_hip(mirror, addrs, batch=B, query_len=T, block_size=bs,
                                                       max_pages=max_pages, stage_dst=stage, stage_words=2 * B)
        desc.mark(torch.cuda.current_stream(device).cuda_stream)
        want_lists = [lists[r] for r in rows]
        ids, offs = oracle.csr(want_lists)
        wpt, w32, w64, wslots = pack_metadata_hip(dev(ids) if len(ids) else dev([0]), dev(offs), dev(prev),
                                                  dev(app), query_len=T, block_size=bs, max_pages=max_pages)
        assert torch.equal(pt, wpt) and torch.equal(s32, w32) and torch.equal(s64, w64)
        assert torch.equal(slots, wslots), step
        assert stage[:2 * B].cpu().tolist() == cur + sel
        got = mirror.cpu().numpy()
        for r in rows:
            assert got[r, :len(lists[r])].tolist() == lists[r] == shadow[r, :slen[r]].tolist()
    desc.close()
    assert desc.host_ptr is None
    desc.close()  # idempotent


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
