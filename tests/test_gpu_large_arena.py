"""Paged attention on a KV layer larger than 2^32 elements.

The reference's arena (attention.rs:34-104) is one Vec indexed with usize, so
a block id anywhere in the pool is valid.  On a 288 GB MI355X a serving pool
can exceed 2^32 bf16 elements (8.59 GB) per layer (260 GB of KV over a
22-layer model is 11.8 GB per layer), so the kernels form block offsets in 64
bits.  This test allocates a 1,050,000-block bf16 layer (hkv 1, d 128, block
16: 4096 elements per block, 8.6 GB, 4.30e9 elements) and reads sequences
whose tables mix blocks below and above the 2^32-element boundary (including
the pool's last block), through the decode and the prefill kernels, against
the oracle on a compacted copy of the same blocks (block ids remapped,
contents identical).
"""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh
from model_fixtures import bf16_round

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 4, 1, 128, 16
NUM_BLOCKS = 1_050_000
BLK_ELEMS = 2 * BS * HKV * D  # 4096
BOUNDARY = (1 << 32) // BLK_ELEMS  # first block past 2^32 elements


def test_layer_past_2_32_elements(backend):
    be = backend
    assert NUM_BLOCKS * BLK_ELEMS > (1 << 32)
    rng = np.random.default_rng(4242)
    # tables: each sequence interleaves low blocks and blocks past the boundary
    high = rng.choice(np.arange(BOUNDARY, NUM_BLOCKS - 1), 60, replace=False)
    high = np.concatenate([high, [NUM_BLOCKS - 1]])
    low = rng.choice(BOUNDARY - 1, 60, replace=False)
    ctxs = [300, 517, 96, 1]
    tables, pool = [], list(np.concatenate([high, low]))
    rng.shuffle(pool)
    pool.remove(NUM_BLOCKS - 1)
    pool.insert(0, NUM_BLOCKS - 1)
    cur = 0
    for c in ctxs:
        nb = -(-c // BS)
        tables.append(np.asarray(pool[cur:cur + nb], np.uint32))
        cur += nb
    used = np.unique(np.concatenate(tables))
    assert (used >= BOUNDARY).any() and (used < BOUNDARY).any()
    # block contents, compact copy for the oracle
    content = bf16_round(rng.standard_normal((len(used), BLK_ELEMS), dtype=np.float32))
    remap = {int(b): i for i, b in enumerate(used)}
    compact_tables = [np.asarray([remap[int(b)] for b in t], np.uint32) for t in tables]

    kv = oh.kv_layout(1, NUM_BLOCKS, BS, HKV, D, oh.BF16)
    print(f"[large arena] allocating {NUM_BLOCKS * BLK_ELEMS * 2 / 1e9:.2f} GB", flush=True)
    arena = be.alloc(NUM_BLOCKS * BLK_ELEMS * 2)
    bits = oh.f32_to_bf16_bits(content)
    for i, b in enumerate(used):
        oh._check(be.lib.orion_hip_memcpy_h2d(be.handle, arena.ptr + int(b) * BLK_ELEMS * 2,
                                              bits[i].ctypes.data, BLK_ELEMS * 2))
    offs = np.zeros(len(ctxs) + 1, np.int64)
    offs[1:] = np.cumsum([len(t) for t in tables])
    ids = np.concatenate(tables).astype(np.uint32)
    cids = np.concatenate(compact_tables).astype(np.uint32)
    dims_c = (1, len(used), BS, HKV, D)
    flat_c = content.reshape(-1)
    dbo, dbi = be.to_device(offs), be.to_device(ids)

    # decode: one row per sequence at ctx - 1
    pos = (np.asarray(ctxs) - 1).astype(np.uint32)
    rs = np.arange(len(ctxs), dtype=np.int32)
    q = rng.standard_normal((len(ctxs), HQ * D), dtype=np.float32)
    bq, bp, br, bout = be.to_device(q), be.to_device(pos), be.to_device(rs), be.alloc(q.nbytes)
    plan = oh.DecodePlan(be, pos, rs, offs, ids, HQ, HKV, D, BS)
    print("[large arena] decode", flush=True)
    oh.paged_attention_decode(be, kv, arena.ptr, 0, bq.ptr, len(ctxs), HQ, bp.ptr, br.ptr,
                              dbo.ptr, dbi.ptr, plan, bout.ptr)
    got = bout.download(np.float32, q.shape)
    plan.close()
    want = orc.paged_attention_rows(flat_c, dims_c, 0, HQ, q, pos, rs, offs, cids)
    err = float(np.abs(got - want).max())
    print(f"[large arena] decode max abs err {err:.2e}", flush=True)
    assert err <= 1e-2
    for b in (bq, bp, br, bout):
        b.free()

    # prefill: the last 256 positions of sequence 1 (517 keys) as one chunk
    cnt, first = 256, ctxs[1] - 256
    qp = bf16_round(rng.standard_normal((cnt, HQ * D), dtype=np.float32))
    bq, bout = be.to_device(qp), be.alloc(qp.nbytes)
    pst, pcnt = be.to_device(np.zeros(1, np.int32)), be.to_device(np.full(1, cnt, np.int32))
    pfp = be.to_device(np.full(1, first, np.uint32))
    pbo = be.to_device(offs[1:2].astype(np.int64))
    print("[large arena] prefill", flush=True)
    oh.paged_attention_prefill(be, kv, arena.ptr, 0, bq.ptr, HQ, 1, pst.ptr, pcnt.ptr, pfp.ptr,
                               pbo.ptr, dbi.ptr, cnt, ctxs[1], bout.ptr, hilo=True)
    got = bout.download(np.float32, qp.shape)
    ppos = np.arange(first, first + cnt, dtype=np.uint32)
    want = orc.paged_attention_rows(flat_c, dims_c, 0, HQ, qp, ppos,
                                    np.full(cnt, 1, np.int32), offs, cids)
    err = float(np.abs(got - want).max())
    print(f"[large arena] prefill max abs err {err:.2e}", flush=True)
    assert err <= 1e-3
    for b in (bq, bout, pst, pcnt, pfp, pbo, dbo, dbi, arena):
        b.free()
