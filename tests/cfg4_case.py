"""benchmark config 4 (full decode step of a random-init TinyLlama-1.1B-shape
model): the batch the bench decodes and the synthetic weights it runs on.

* ``cfg4_case`` draws the bench's exact batch: 32 sequences with prompt
  lengths U[16, 1024], random token ids, block tables scattered over a pool
  1.1x the blocks needed for prompt + 64 steps (the same numpy Generator
  calls, in the same order, as ``bench.decode_e2e``).
* ``synthetic_weight_np`` restates the library's counter-based weight generator
  (``orion_hip_synthetic_value`` / ``orion_hip_model_init_synthetic``) in
  numpy: splitmix64 of a per-tensor key plus the element index, the sum of the
  hash's four 16-bit fields (Irwin-Hall) centred and scaled to the requested
  standard deviation, rounded to bf16 (nearest even) and widened back to f32.
  Norm weights are ones.  ``tests/test_cfg4_golden.py`` checks it, and the
  oracle's C restatement used to fill models, against the library's host entry
  point element by element on samples.
"""
import numpy as np

TINYLLAMA = dict(L=22, H=2048, hq=32, hkv=4, d=64, F=5632, V=32000, eps=1e-5, theta=10000.0,
                 max_pos=2048)
SEED = 20261204
STD = 0.02

# weight ids (include/orion_hip.h ORION_W_*)
W_EMBED, W_FINAL_NORM, W_LM_HEAD, W_INPUT_NORM = 0, 1, 2, 3
W_Q, W_K, W_V, W_O, W_POST_NORM, W_GATE, W_UP, W_DOWN = 4, 5, 6, 7, 11, 12, 13, 14

_IRWIN_HALL_SD = np.float32(37837.2265625)  # 65536 / sqrt(3), rounded to f32


class Cfg4Case:
    def __init__(self, lens, tables, num_blocks, prompts, steps):
        self.lens, self.tables, self.num_blocks = lens, tables, num_blocks
        self.prompts, self.steps = prompts, steps
        self.seqs = len(lens)


def cfg4_case(seed=SEED, seqs=32, steps=64):
    rng = np.random.default_rng(seed)
    lens = rng.integers(16, 1025, size=seqs)
    bs = 16
    need = [-(-int(n + steps) // bs) for n in lens]
    num_blocks = int(sum(need) * 1.1) + 8
    perm = rng.permutation(num_blocks)
    tables, cur = [], 0
    for nb in need:
        tables.append(perm[cur:cur + nb].tolist())
        cur += nb
    prompts = [rng.integers(0, TINYLLAMA["V"], size=int(n)).tolist() for n in lens]
    return Cfg4Case([int(n) for n in lens], tables, num_blocks, prompts, steps)


def _splitmix64(x):
    with np.errstate(over="ignore"):
        x = x + np.uint64(0x9E3779B97F4A7C15)
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return x ^ (x >> np.uint64(31))


def synthetic_key(seed, which, layer):
    lay = layer if which >= W_INPUT_NORM else -1
    k = (np.uint64(seed) ^ (np.uint64(which + 1) << np.uint64(48))
         ^ (np.uint64((lay + 1) & 0xFFFFFFFFFFFFFFFF) << np.uint64(24)))
    return _splitmix64(np.asarray(k, dtype=np.uint64))


def _f32_to_bf16_f32(v):
    u = v.view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32)
    return (r << 16).view(np.float32)


def synthetic_weight_np(seed, which, layer, count, std=STD, chunk=1 << 24):
    """f32 values (bf16-exact) of weight `which` of `layer`, logical row-major order
    (numpy; the oracle's ``synthetic_weight`` is the fast C restatement)."""
    if which in (W_FINAL_NORM, W_INPUT_NORM, W_POST_NORM):
        return np.ones(count, np.float32)
    mul = np.float32(np.float32(std) / _IRWIN_HALL_SD)
    key = synthetic_key(seed, which, layer)
    out = np.empty(count, np.float32)
    for s in range(0, count, chunk):
        idx = np.arange(s, min(count, s + chunk), dtype=np.uint64)
        with np.errstate(over="ignore"):
            h = _splitmix64(key + idx)
        f = ((h & np.uint64(0xFFFF)) + ((h >> np.uint64(16)) & np.uint64(0xFFFF))
             + ((h >> np.uint64(32)) & np.uint64(0xFFFF)) + (h >> np.uint64(48))).astype(np.int32)
        v = (f - np.int32(131070)).astype(np.float32) * mul
        out[s:s + len(idx)] = _f32_to_bf16_f32(v)
    return out


def layer_weight_shapes(cfg=TINYLLAMA):
    H, F = cfg["H"], cfg["F"]
    qd, kvd = cfg["hq"] * cfg["d"], cfg["hkv"] * cfg["d"]
    return [(W_INPUT_NORM, H), (W_Q, qd * H), (W_K, kvd * H), (W_V, kvd * H), (W_O, H * qd),
            (W_POST_NORM, H), (W_GATE, F * H), (W_UP, F * H), (W_DOWN, H * F)]


def oracle_tinyllama(orc, num_blocks, seed=SEED, cfg=TINYLLAMA, block_size=16, kv_bf16=False):
    """An OracleTransformer of the config-4 shape holding the synthetic weights."""
    m = orc.OracleTransformer(cfg["L"], cfg["H"], cfg["hq"], cfg["hkv"], cfg["d"], cfg["F"],
                              cfg["V"], cfg["max_pos"], cfg["eps"], cfg["theta"], False, False,
                              num_blocks, block_size, kv_bf16=kv_bf16)
    H, V = cfg["H"], cfg["V"]
    for wid, n in [(W_EMBED, V * H), (W_LM_HEAD, V * H), (W_FINAL_NORM, H)]:
        m.set_weight(wid, -1, orc.synthetic_weight(seed, wid, -1, n, STD))
    for l in range(cfg["L"]):
        for wid, n in layer_weight_shapes(cfg):
            m.set_weight(wid, l, orc.synthetic_weight(seed, wid, l, n, STD))
    return m
