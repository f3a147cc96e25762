"""In-place streaming KV cache (sr_dit.kv_ring.KVRing): host bookkeeping on the CPU.

The reference's cache update is "concatenate the cache with the chunk, keep
the last kv_len frames" (video_refiner/wan/modules/sr_dit/attention.py:
1506-1510, :964-974).  These tests drive a ring and that rule side by side
over chunk sequences that wrap the ring several times and compare:
  * the cached frames in order (``logical``) with the reference's cache tensor;
  * every logical KV frame of the next call, read at ``physical_frame`` (the
    kernels' mapping), with the frame the reference's concatenation holds there.
"""
import pytest
import torch

from sr_dit.kv_ring import KVRing

L, N, D = 6, 2, 4


def _chunk(seed, frames, batch):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(batch, frames * L, N, D, generator=g)


def _reference_step(cache, new, kv_len):
    full = new if cache is None else torch.cat([cache, new], 1)
    frames = full.shape[1] // L
    return full, (full if frames <= kv_len else full[:, -kv_len * L:])


def _frame(t, f):
    return t[:, f * L:(f + 1) * L]


@pytest.mark.parametrize("kv_len,chunk,anchor", [(4, 2, 0), (5, 3, 0), (9, 3, 12), (2, 3, 0),
                                                 (1, 1, 5), (6, 2, 3)])
def test_ring_matches_cat_and_tail(kv_len, chunk, anchor):
    batch = 2
    ring = KVRing(batch, kv_len, chunk, L, N, D, anchor_tokens=anchor, dtype=torch.float32,
                  device="cpu")
    cache_k = cache_v = None
    for step in range(9):
        f_cur = chunk if step % 4 else max(1, chunk - 1)  # some short chunks
        k, v = _chunk(2 * step, f_cur, batch), _chunk(2 * step + 1, f_cur, batch)
        for i in range(batch):
            ring.write_current(i, k[i], v[i])
        full_k, new_k = _reference_step(cache_k, k, kv_len)
        full_v, new_v = _reference_step(cache_v, v, kv_len)
        f_kv = full_k.shape[1] // L
        assert ring.cached + f_cur == f_kv
        for f in range(f_kv):  # what the kernel reads for logical frame f
            p = ring.physical_frame(f)
            got_k = ring.k[:, anchor + p * L:anchor + (p + 1) * L]
            got_v = ring.v[:, anchor + p * L:anchor + (p + 1) * L]
            assert torch.equal(got_k, _frame(full_k, f)), (step, f)
            assert torch.equal(got_v, _frame(full_v, f)), (step, f)
        ring.commit(f_cur)
        cache_k, cache_v = new_k, new_v
        assert ring.cached == cache_k.shape[1] // L
        assert int(ring.head_dev[0]) == ring.head
        for i in range(batch):
            lk, lv = ring.logical(i)
            assert torch.equal(lk, cache_k[i]) and torch.equal(lv, cache_v[i])


def test_ring_load_reset_and_anchor_prefix():
    ring = KVRing(1, 3, 2, L, N, D, anchor_tokens=4, dtype=torch.float32, device="cpu")
    pre = _chunk(7, 5, 1)
    ring.load(pre, pre * 2)
    lk, lv = ring.logical(0)
    assert torch.equal(lk, pre[0, -3 * L:]) and torch.equal(lv, 2 * pre[0, -3 * L:])
    ak = torch.arange(4 * N * D, dtype=torch.float32).view(4, N, D)
    ring.write_anchor(0, ak, -ak)
    assert torch.equal(ring.k[0, :4], ak) and torch.equal(ring.v[0, :4], -ak)
    # the prefix is outside the HR region: loading and committing leave it alone
    ring.write_current(0, _chunk(8, 2, 1)[0], _chunk(9, 2, 1)[0])
    ring.commit(2)
    assert torch.equal(ring.k[0, :4], ak)
    ring.reset()
    assert ring.cached == 0 and ring.head == 0 and ring.logical(0)[0].shape[0] == 0


def test_in_place_producer_skips_copy():
    ring = KVRing(1, 4, 2, L, N, D, dtype=torch.float32, device="cpu")
    ck = ring.current_k(0)
    ck.copy_(_chunk(3, 2, 1)[0])
    before = ck.clone()
    ring.write_current(0, ck, ring.current_v(0))  # same storage: nothing to do
    assert torch.equal(ring.current_k(0), before)


def test_ring_rejects_bad_arguments():
    with pytest.raises(ValueError):
        KVRing(1, 0, 2, L, N, D, device="cpu")
    with pytest.raises(ValueError):
        KVRing(1, None, 2, L, N, D, device="cpu")
    ring = KVRing(1, 4, 2, L, N, D, anchor_tokens=3, dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError):
        ring.write_current(0, _chunk(1, 3, 1)[0], _chunk(2, 3, 1)[0])  # 3 frames > 2
    with pytest.raises(ValueError):
        ring.write_anchor(0, torch.zeros(4, N, D), torch.zeros(4, N, D))  # 4 > 3 tokens
    with pytest.raises(ValueError):
        ring.commit(3)
    with pytest.raises(ValueError):
        ring.load(torch.zeros(1, L + 1, N, D), torch.zeros(1, L + 1, N, D))


def test_op_rejects_ring_with_cache_tensors():
    from sr_dit import attention as att
    ring = KVRing(1, 4, 2, L, N, D, dtype=torch.float32, device="cpu")
    q = torch.zeros(1, 2 * L, N, D)
    with pytest.raises(ValueError, match="either kv_ring"):
        att.mask_free_window_attention(q, q, q, [[2, 2, 3]], pre_cache_k=q, pre_cache_v=q,
                                       kv_ring=ring, block_t=2)
    with pytest.raises(ValueError, match="kv_len"):
        att.mask_free_window_attention(q, q, q, [[2, 2, 3]], kv_len=3, kv_ring=ring, block_t=2)
    with pytest.raises(ValueError, match="does not fit"):
        att.mask_free_window_attention(torch.zeros(1, 3 * L, N, D), torch.zeros(1, 3 * L, N, D),
                                       torch.zeros(1, 3 * L, N, D), [[3, 2, 3]], kv_ring=ring,
                                       block_t=2)
