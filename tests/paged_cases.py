"""Seeded paged-attention workloads (benchmark configs 1 and 2 and edge cases)
shared by the GPU parity tests, the golden-fixture generator and bench.py."""
import numpy as np


class PagedCase:
    """Sequences with context lengths `ctxs`, block tables drawn from a
    seeded permutation of a pool of `num_blocks`, and one query row per
    sequence at position ctx - 1 (decode).  K/V pool entries are N(0, 1)
    (also the never-referenced blocks), stored in `dtype` ('f32' | 'bf16').
    With `rope_theta`, every cached K vector and every query is rotated by
    RoPE at its position first (rotate-half, the reference's f32 table and
    formula, tensor.rs:228-298), as the model does before caching."""

    def __init__(self, seed, ctxs, hq, hkv, d, block_size, num_blocks=None, dtype="f32",
                 pool_factor=1.25, disjoint=True, head_major=False, rope_theta=None):
        rng = np.random.default_rng(seed)
        self.ctxs = np.asarray(ctxs, dtype=np.int64)
        self.S = len(ctxs)
        self.hq, self.hkv, self.d, self.bs = hq, hkv, d, block_size
        self.dtype = dtype
        self.head_major = head_major  # device arena block order (the oracle's is reference)
        need = [-(-int(c) // block_size) for c in self.ctxs]
        total = sum(need)
        self.num_blocks = int(num_blocks or int(np.ceil(pool_factor * total)) or 1)
        perm = rng.permutation(self.num_blocks)
        tables, cur = [], 0
        for nb in need:
            if disjoint:
                tables.append(perm[cur:cur + nb].astype(np.uint32))
                cur += nb
            else:
                tables.append(rng.integers(0, self.num_blocks, nb).astype(np.uint32))
        self.tables = tables
        self.bt_offsets = np.zeros(self.S + 1, np.int64)
        self.bt_offsets[1:] = np.cumsum(need)
        self.bt_ids = np.concatenate(tables) if total else np.zeros(1, np.uint32)
        n_el = self.num_blocks * 2 * block_size * hkv * d
        arena = rng.standard_normal(n_el, dtype=np.float32)
        self.q = rng.standard_normal((self.S, hq * d), dtype=np.float32)
        self.positions = (self.ctxs - 1).astype(np.uint32)
        self.rope_theta = rope_theta
        if rope_theta is not None and total:
            import oracle as orc
            table = orc.RopeTable(d, int(self.ctxs.max()), rope_theta)
            k = arena.reshape(self.num_blocks, 2, block_size, hkv, d)
            for t, c in zip(tables, self.ctxs):
                p = np.arange(int(c))
                blk, slot = t[p // block_size], p % block_size
                k[blk, 0, slot] = rope_rotate(k[blk, 0, slot], table.cos[p], table.sin[p])
            self.q = rope_rotate(self.q.reshape(self.S, hq, d), table.cos[self.positions],
                                 table.sin[self.positions]).reshape(self.S, hq * d)
        if dtype == "bf16":
            from model_fixtures import bf16_round
            arena = bf16_round(arena)
        self.arena_f32 = arena  # exact values the device holds, widened to f32
        self.row_seq = np.arange(self.S, dtype=np.int32)

    def share_prefixes(self, groups):
        """Prefix sharing: for each (rows, nblocks) in `groups`, the first
        `nblocks` table entries of every listed row become those of the
        group's first row (identical leading block ids, as prefix caching
        produces).  Each row must hold at least that many blocks."""
        for rows, nb in groups:
            lead = self.tables[rows[0]][:nb].copy()
            for r in rows[1:]:
                assert len(self.tables[r]) >= nb
                self.tables[r] = np.concatenate([lead, self.tables[r][nb:]]).astype(np.uint32)
        self.bt_ids = np.concatenate(self.tables)
        return self

    def dims(self):
        return (1, self.num_blocks, self.bs, self.hkv, self.d)

    def arena_device(self):
        """The arena in the device layout (reference order unless head_major)."""
        a = self.arena_f32
        if self.head_major:
            a = np.ascontiguousarray(
                a.reshape(self.num_blocks, 2, self.bs, self.hkv, self.d).transpose(0, 3, 1, 2, 4))
        return a.reshape(-1)

    def arena_device_bytes(self):
        if self.dtype == "bf16":
            import orion_hip
            return orion_hip.f32_to_bf16_bits(self.arena_device())
        return self.arena_device()

    def kv_layout(self):
        import orion_hip as oh
        return oh.kv_layout(1, self.num_blocks, self.bs, self.hkv, self.d,
                            oh.BF16 if self.dtype == "bf16" else oh.F32, self.head_major)

    def kv_bytes_read(self):
        esz = 2 if self.dtype == "bf16" else 4
        return int(self.ctxs.sum()) * 2 * self.hkv * self.d * esz

    def oracle(self, positions=None, row_seq=None, q=None):
        import oracle as orc
        return orc.paged_attention_rows(
            self.arena_f32, self.dims(), 0, self.hq, self.q if q is None else q,
            self.positions if positions is None else positions,
            self.row_seq if row_seq is None else row_seq, self.bt_offsets, self.bt_ids)


def rope_rotate(x, cos, sin):
    """apply_rope (tensor.rs:283-298) on [n, heads, d] vectors at n positions:
    (x_i, x_{i+d/2}) -> (x_i c - x_{i+d/2} s, x_i s + x_{i+d/2} c) in f32;
    cos/sin are [n, d/2] rows of the reference's RopeTable."""
    half = x.shape[-1] // 2
    c, s = cos[:, None, :].astype(np.float32), sin[:, None, :].astype(np.float32)
    x0, x1 = x[..., :half], x[..., half:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1).astype(np.float32)


def cfg1(seed=20261201):
    """benchmark config 1: 4 seqs, ctx U[1,512], bs 16, 8q/2kv, d 64, f32, 256-block pool."""
    rng = np.random.default_rng(seed)
    ctxs = rng.integers(1, 513, size=4)
    return PagedCase(seed + 1, ctxs, 8, 2, 64, 16, num_blocks=256, dtype="f32")


def cfg2(seed=20261202, num_seqs=64, head_major=False):
    """benchmark config 2: 64 seqs, ctx U[128,4096], bs 16, 32q/8kv, d 128, bf16 KV,
    pool 1.25x the blocks needed, scattered tables; Q and cached K rotated by
    RoPE (theta 500000) at their positions before caching."""
    rng = np.random.default_rng(seed)
    ctxs = rng.integers(128, 4097, size=num_seqs)
    return PagedCase(seed + 1, ctxs, 32, 8, 128, 16, dtype="bf16", pool_factor=1.25,
                     head_major=head_major, rope_theta=500000.0)


class PrefillCase(PagedCase):
    """Chunked prefill: sequence s has `prefixes[s]` cached tokens plus a new
    chunk of `chunks[s]` rows at consecutive positions prefix .. prefix +
    chunk - 1 (all of whose K/V are already in the arena, as after the KV
    write).  Rows are laid out sequence after sequence.  With bf16 KV the
    queries are bf16-representable too ("bf16 inputs")."""

    def __init__(self, seed, prefixes, chunks, hq, hkv, d, block_size, dtype="bf16",
                 **kw):
        prefixes = np.asarray(prefixes, np.int64)
        chunks = np.asarray(chunks, np.int64)
        super().__init__(seed, prefixes + chunks, hq, hkv, d, block_size, dtype=dtype, **kw)
        rng = np.random.default_rng(seed + 7)
        self.prefixes, self.chunks = prefixes, chunks
        self.row_start = np.zeros(self.S, np.int32)
        self.row_start[1:] = np.cumsum(chunks)[:-1]
        self.row_count = chunks.astype(np.int32)
        self.first_pos = prefixes.astype(np.uint32)
        n = int(chunks.sum())
        self.positions = np.concatenate(
            [np.arange(p, p + c, dtype=np.uint32) for p, c in zip(prefixes, chunks)]) \
            if n else np.zeros(0, np.uint32)
        self.row_seq = np.repeat(np.arange(self.S, dtype=np.int32), chunks)
        q = rng.standard_normal((n, hq * d), dtype=np.float32)
        if dtype == "bf16":
            from model_fixtures import bf16_round
            q = bf16_round(q)
        self.q = q

    def flops(self):
        """Algorithmic flops: 4 * Hq * d per (query row, attended key)."""
        per_seq = self.chunks * self.prefixes + self.chunks * (self.chunks + 1) // 2
        return 4 * self.hq * self.d * int(per_seq.sum())

    def oracle_rows(self, rows):
        """Oracle output for the listed rows only ([len(rows), Hq*d])."""
        rows = np.asarray(rows, np.int64)
        return self.oracle(self.positions[rows], self.row_seq[rows], self.q[rows])


def cfg3(seed=20261203, head_major=False):
    """benchmark config 3: 8 seqs x 512-token chunk on a prefix U[0,7680], bs 16,
    32q/8kv, d 128, bf16 inputs, scattered tables."""
    rng = np.random.default_rng(seed)
    prefixes = rng.integers(0, 7681, size=8)
    return PrefillCase(seed + 1, prefixes, [512] * 8, 32, 8, 128, 16, dtype="bf16",
                       head_major=head_major)


class MixedBatch:
    """A continuous batch mixing prefill chunks and decode rows, with prefix
    sharing (benchmark config 5's structure).  Sequence s has `cached[s]`
    tokens in the cache before this step and contributes `counts[s]` new rows
    at positions cached[s] .. cached[s] + counts[s] - 1.  Sharing sequences
    start with the same `prefix` tokens, stored once: their tables begin with
    the same block ids (refcount > 1 in orion-kv-cache terms).  The rest of
    each context is lognormal (median `median`, shape `sigma`), capped so the
    whole context stays <= `cap`."""

    def __init__(self, seed, n_prefill, chunk, n_decode, share_frac, prefix, median, sigma, cap,
                 block_size, vocab):
        rng = np.random.default_rng(seed)
        S = n_prefill + n_decode
        self.S, self.bs = S, block_size
        order = rng.permutation(S)
        is_prefill = np.zeros(S, bool)
        is_prefill[order[:n_prefill]] = True
        shares = np.zeros(S, bool)
        shares[rng.permutation(S)[:int(round(share_frac * S))]] = True
        own = np.minimum(np.round(rng.lognormal(np.log(median), sigma, S)).astype(np.int64), cap)
        self.counts = np.where(is_prefill, chunk, 1).astype(np.int64)
        base = np.where(shares, prefix, 0)
        self.cached = np.minimum(base + own, cap - self.counts)
        self.cached = np.maximum(self.cached, base)  # a sharing context keeps the whole prefix
        self.ctx = self.cached + self.counts
        self.is_prefill, self.shares = is_prefill, shares
        # block tables: the shared prefix blocks first, then private blocks
        nshared = -(-prefix // block_size)
        shared_ids = np.arange(nshared, dtype=np.uint32)
        nxt = nshared
        tables = []
        for s in range(S):
            need = -(-int(self.ctx[s]) // block_size)
            if shares[s]:
                priv = need - nshared
                t = np.concatenate([shared_ids, np.arange(nxt, nxt + priv, dtype=np.uint32)])
                nxt += priv
            else:
                t = np.arange(nxt, nxt + need, dtype=np.uint32)
                nxt += need
            tables.append(t)
        # scatter the private blocks over the pool (the shared ones stay put)
        self.num_blocks = int(nxt)
        perm = np.concatenate([shared_ids, nshared + rng.permutation(nxt - nshared)]).astype(np.uint32)
        self.tables = [perm[t] for t in tables]
        self.positions = np.concatenate(
            [np.arange(self.cached[s], self.ctx[s], dtype=np.uint32) for s in range(S)])
        self.tokens = rng.integers(0, vocab, len(self.positions)).astype(np.uint32)
        self.row_seq = np.repeat(np.arange(S, dtype=np.int32), self.counts)

    def decode_rows(self):
        starts = np.concatenate([[0], np.cumsum(self.counts)[:-1]])
        return starts[~self.is_prefill]

    def kv_bytes(self, hkv, d, esz=2):
        """(unique, logical) K+V bytes one layer's attention reads for the
        decode rows: blocks touched counted once vs every attended token."""
        blk = hkv * d * 2 * esz * self.bs
        dec = ~self.is_prefill
        uniq = set()
        for s in np.nonzero(dec)[0]:
            uniq.update(self.tables[s][:-(-int(self.ctx[s]) // self.bs)].tolist())
        logical = int(self.ctx[dec].sum()) * hkv * d * 2 * esz
        return len(uniq) * blk, logical


def cfg5_batch(vocab, seed=20261205):
    """benchmark config 5: 8 prefill chunks of 256 + 192 decodes; half of the
    200 sequences share a 2048-token prefix; other context lognormal (median
    1024; shape 1.0, not given by the config) capped at 16384; block 16."""
    return MixedBatch(seed, 8, 256, 192, 0.5, 2048, 1024, 1.0, 16384, 16, vocab)
