"""benchmark config 5 at full size: a mixed continuous batch with prefix sharing
at the Qwen2-7B layer shape (28 query / 4 KV heads, head_dim 128, hidden
3584, QKV bias, bf16): 8 prefill chunks of 256 tokens and 192 decode rows
over 200 sequences, half of them sharing a 2048-token prefix through
identical leading block ids, other contexts lognormal (median 1024) capped at
16384, block 16 (tests/paged_cases.py cfg5_batch, the bench's batch).

* Attention (attention.rs:219-295): decode attention over all 192 decode rows
  and chunked-prefill attention over sampled rows of every chunk (first and
  last row of each chunk plus random rows), against the oracle on the same
  bf16 arena; the rows include shared-prefix sequences and the longest
  (16,384-token) context.
* One layer forward (transformer.rs:230-442) on the whole batch, against the
  oracle run on a subset of the sequences (the reference's batching
  independence makes the subset's logits those of the full batch): the two
  prefill chunks that continue a shared prefix, the longest decode sequence,
  and decode sequences with and without the shared prefix.  The oracle
  rounds K/V to bf16 when writing, as the device arena does.
"""
import numpy as np
import pytest

import oracle as orc
import orion_hip as oh
from model_fixtures import bf16_round
from paged_cases import cfg5_batch

pytestmark = pytest.mark.gpu

HQ, HKV, D, H, F, V = 28, 4, 128, 3584, 18944, 1024


@pytest.fixture(scope="module")
def mixed():
    b = cfg5_batch(V)
    rng = np.random.default_rng(55)
    arena = bf16_round(rng.standard_normal(b.num_blocks * 2 * b.bs * HKV * D,
                                           dtype=np.float32))
    return b, arena


def tables_csr(b):
    offs = np.zeros(b.S + 1, np.int64)
    offs[1:] = np.cumsum([len(t) for t in b.tables])
    return offs, np.concatenate(b.tables).astype(np.uint32)


def test_cfg5_attention_full_size(backend, mixed):
    b, arena = mixed
    be = backend
    kv = oh.kv_layout(1, b.num_blocks, b.bs, HKV, D, oh.BF16)
    offs, ids = tables_csr(b)
    rng = np.random.default_rng(56)
    dims = (1, b.num_blocks, b.bs, HKV, D)
    darena = be.to_device(oh.f32_to_bf16_bits(arena))
    dbo, dbi = be.to_device(offs), be.to_device(ids)
    # decode rows: one per decode sequence at ctx - 1
    dec = np.nonzero(~b.is_prefill)[0]
    pos_d = (b.ctx[dec] - 1).astype(np.uint32)
    rs_d = dec.astype(np.int32)
    q_d = rng.standard_normal((len(dec), HQ * D), dtype=np.float32)
    print(f"[cfg5 attention] decode {len(dec)} rows, longest ctx {int(b.ctx[dec].max())}",
          flush=True)
    bq, bp, br, bout = (be.to_device(q_d), be.to_device(pos_d), be.to_device(rs_d),
                        be.alloc(q_d.nbytes))
    plan = oh.DecodePlan(be, pos_d, rs_d, offs, ids, HQ, HKV, D, b.bs)
    oh.paged_attention_decode(be, kv, darena.ptr, 0, bq.ptr, len(dec), HQ, bp.ptr, br.ptr,
                              dbo.ptr, dbi.ptr, plan, bout.ptr)
    got = bout.download(np.float32, q_d.shape)
    plan.close()
    want = orc.paged_attention_rows(arena, dims, 0, HQ, q_d, pos_d, rs_d, offs, ids)
    err = float(np.abs(got - want).max())
    print(f"[cfg5 attention] decode max abs err {err:.2e}", flush=True)
    assert err <= 1e-2
    assert b.shares[dec].any() and (~b.shares[dec]).any() and int(b.ctx[dec].max()) == 16384
    for buf in (bq, bp, br, bout):
        buf.free()
    # prefill chunks: 256 consecutive rows per chunk, sequence after sequence
    pf = np.nonzero(b.is_prefill)[0]
    n = 256 * len(pf)
    q_p = bf16_round(rng.standard_normal((n, HQ * D), dtype=np.float32))
    pos_p = np.concatenate([np.arange(b.cached[s], b.ctx[s]) for s in pf]).astype(np.uint32)
    rs_p = np.repeat(pf, 256).astype(np.int32)
    bq, bout = be.to_device(q_p), be.alloc(q_p.nbytes)
    pst = be.to_device((np.arange(len(pf)) * 256).astype(np.int32))
    pcnt = be.to_device(np.full(len(pf), 256, np.int32))
    pfp = be.to_device(b.cached[pf].astype(np.uint32))
    pbo = be.to_device(offs[pf].astype(np.int64))
    rows = sorted({r for c in range(len(pf)) for r in (256 * c, 256 * c + 255)}
                  | set(rng.choice(n, 48, replace=False).tolist()))
    rows = np.asarray(rows)
    want = orc.paged_attention_rows(arena, dims, 0, HQ, q_p[rows], pos_p[rows], rs_p[rows],
                                    offs, ids)
    for hilo, tol in ((True, 1e-3), (False, 1e-2)):
        print(f"[cfg5 attention] prefill {len(pf)} chunks hilo={hilo}, {len(rows)} rows checked",
              flush=True)
        oh.paged_attention_prefill(be, kv, darena.ptr, 0, bq.ptr, HQ, len(pf), pst.ptr,
                                   pcnt.ptr, pfp.ptr, pbo.ptr, dbi.ptr, 256, int(b.ctx.max()),
                                   bout.ptr, hilo=hilo)
        got = bout.download(np.float32, q_p.shape)
        err = float(np.abs(got[rows] - want).max())
        print(f"[cfg5 attention] prefill hilo={hilo} max abs err {err:.2e}", flush=True)
        assert err <= tol, (hilo, err)
    for buf in (darena, dbo, dbi, bq, bout, pst, pcnt, pfp, pbo):
        buf.free()


def test_cfg5_layer_forward_matches_oracle_on_a_subset(backend, mixed):
    b, arena = mixed
    be = backend
    meta = oh.ModelMetadata(hidden_size=H, num_layers=1, num_attention_heads=HQ,
                            num_kv_heads=HKV, head_dim=D, vocab_size=V, intermediate_size=F,
                            max_position_embeddings=16640, rope_theta=1e6, rms_norm_eps=1e-6,
                            architecture="qwen2", tied_lm_head=False)
    m = oh.HipTransformerModel(meta, b.num_blocks, b.bs, be, oh.BF16)
    m.init_synthetic(20261205, 0.02)
    ptr, nbytes = m.kv_arena()
    bits = oh.f32_to_bf16_bits(arena)
    assert bits.nbytes == nbytes
    oh._check(be.lib.orion_hip_memcpy_h2d(be.handle, ptr, bits.ctypes.data, bits.nbytes))
    print(f"[cfg5 layer] forward {len(b.positions)} rows over {b.S} sequences", flush=True)
    g = m.forward(oh.ForwardBatch(b.tokens.tolist(), b.positions.tolist(), list(range(b.S)),
                                  b.counts.tolist(), b.ctx.tolist(),
                                  [t.tolist() for t in b.tables], True)).logits
    # the subset: prefill chunks on a shared prefix (two), the longest decode
    # sequence, two sharing and two private decode sequences
    pf = [s for s in np.nonzero(b.is_prefill)[0] if b.shares[s]][:2]
    dec = np.nonzero(~b.is_prefill)[0]
    longest = int(dec[np.argmax(b.ctx[dec])])
    share_d = [int(s) for s in dec if b.shares[s] and s != longest][:2]
    own_d = [int(s) for s in dec if not b.shares[s] and s != longest][:2]
    subset = sorted(set([int(s) for s in pf] + [longest] + share_d + own_d))
    om = orc.OracleTransformer(1, H, HQ, HKV, D, F, V, 16640, 1e-6, 1e6, True, False,
                               b.num_blocks, b.bs, kv_bf16=True)
    qd, kvd = HQ * D, HKV * D
    for wid, cnt in [(oh.W_EMBED, V * H), (oh.W_LM_HEAD, V * H), (oh.W_FINAL_NORM, H)]:
        om.set_weight(wid, -1, m.download_weight(wid, -1, cnt))
    for wid, cnt in [(oh.W_INPUT_NORM, H), (oh.W_Q, qd * H), (oh.W_K, kvd * H),
                     (oh.W_V, kvd * H), (oh.W_O, H * qd), (oh.W_Q_BIAS, qd),
                     (oh.W_K_BIAS, kvd), (oh.W_V_BIAS, kvd), (oh.W_POST_NORM, H),
                     (oh.W_GATE, F * H), (oh.W_UP, F * H), (oh.W_DOWN, H * F)]:
        om.set_weight(wid, 0, m.download_weight(wid, 0, cnt))
    om.kv()[:] = arena
    starts = np.concatenate([[0], np.cumsum(b.counts)[:-1]])
    toks, pos = [], []
    for s in subset:
        r0, c = int(starts[s]), int(b.counts[s])
        toks += b.tokens[r0:r0 + c].tolist()
        pos += b.positions[r0:r0 + c].tolist()
    print(f"[cfg5 layer] oracle on sequences {subset}", flush=True)
    o = om.forward(toks, pos, [int(b.counts[s]) for s in subset],
                   [int(b.ctx[s]) for s in subset], [b.tables[s].tolist() for s in subset])
    err = float(np.abs(g[subset] - o).max() / np.abs(o).max())
    print(f"[cfg5 layer] relative logit error {err:.2e}", flush=True)
    assert err <= 2e-3, err
    abs_err = float(np.abs(g[subset] - o).max())
    for gr, orow in zip(g[subset], o):
        if int(np.argmax(gr)) != orc.argmax(orow):
            top2 = np.sort(orow)[-2:]
            assert top2[1] - top2[0] <= 2 * abs_err
    om.close()
    m.close()
