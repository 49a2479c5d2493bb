"""Seeded synthetic workloads of the benchmark configurations.

cfg1  one mixed iteration: 4 decode sequences with cached contexts 17, 133,
      512, 1000 (KV seeded N(0,1)) + one 60-token prefill chunk -> M = 64
cfg3  ragged attention: 64 decode sequences, KV length
      clip(round(exp(ln 1024 + sigma z)), 32, 8192) with sigma = 1.0, plus two
      512-token causal chunks at offsets 0 and 1536
cfg4  serve load: C requests, prompt length U[64, 2048] of uniform token ids,
      max_new 64, greedy
All draws come from numpy's PCG64 seeded generator.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

CFG1_CONTEXTS = (17, 133, 512, 1000)
CFG1_PREFILL = 60


def seeded_kv(rng: np.random.Generator, layers: int, n: int, nkv: int, hd: int):
    k = rng.standard_normal((layers, n, nkv, hd), dtype=np.float32)
    v = rng.standard_normal((layers, n, nkv, hd), dtype=np.float32)
    return k, v


@dataclass
class Cfg1:
    contexts: tuple
    kv: list            # [(k, v)] per decode sequence
    dec_tokens: list    # input token of each decode row
    pre_tokens: list    # 60 prompt tokens of the prefill chunk


def cfg1(cfg, seed: int = 1) -> Cfg1:
    rng = np.random.default_rng(seed)
    kv = [seeded_kv(rng, cfg.layers, n, cfg.n_kv, cfg.head_dim) for n in CFG1_CONTEXTS]
    dec = rng.integers(0, cfg.vocab, size=len(CFG1_CONTEXTS)).tolist()
    pre = rng.integers(0, cfg.vocab, size=CFG1_PREFILL).tolist()
    return Cfg1(CFG1_CONTEXTS, kv, dec, pre)


def cfg1_rows(w: Cfg1, dec_slots, pre_slot):
    rows = [(s, n, t, 0, 1) for s, n, t in zip(dec_slots, w.contexts, w.dec_tokens)]
    P = len(w.pre_tokens)
    rows += [(pre_slot, p, t, 1, 1 if p == P - 1 else 0) for p, t in enumerate(w.pre_tokens)]
    return rows


def cfg3_lengths(seed: int = 3, n: int = 64, sigma: float = 1.0):
    rng = np.random.default_rng(seed)
    z = rng.standard_normal(n)
    return np.clip(np.round(np.exp(np.log(1024.0) + sigma * z)), 32, 8192).astype(int).tolist()


def cfg4_requests(C: int, seed: int = 4, vocab: int = 151936, lo: int = 64, hi: int = 2048):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=C)
    return [rng.integers(0, vocab, size=int(n)).astype(np.int32) for n in lens]


def successor_model(model, embed_std: float, seed: int = 5):
    """Turn a synthetic model (in place) into the large-margin variant used
    where greedy streams must not hinge on near-ties: the embedding drawn
    N(0, embed_std) instead of N(0, 0.02) (the seeded draws scaled), and an
    untied lm_head whose row v is embedding row perm[v] for a seeded
    permutation.  While the input token's embedding dominates the residual,
    the logit of v is largest where perm[v] is the input token, so greedy
    decoding follows the chain t -> inv[t] with a top-2 margin of several
    sigma (the random-init model's margins are hundredths of sigma), and the
    rest of the network still moves every logit.  Measured on the CPU
    oracle: 28-layer 0.8B class at embed_std 1.0, every step of a 40-token
    prompt follows the chain with margins 2.3 to 5.1 sigma; the 2-layer
    27B class needs 16.0 (the wider layers add more to the residual).
    Returns (perm, inv); the model keeps the lm_head array alive."""
    import ctypes as C
    cfg = model.cfg
    V, H = cfg.vocab, cfg.hidden
    emb = np.ctypeslib.as_array(model.ptr.contents.embed, shape=(V, H))
    emb *= np.float32(embed_std / 0.02)
    perm = np.random.default_rng(seed).permutation(V)
    lm = np.ascontiguousarray(emb[perm])
    model._successor_lm_head = lm
    model.ptr.contents.lm_head = lm.ctypes.data_as(C.POINTER(C.c_float))
    inv = np.empty(V, np.int64)
    inv[perm] = np.arange(V)
    return perm, inv


def successor_chain(inv, start: int, n: int):
    """n tokens of the successor chain from start: start, inv[start], ..."""
    out = [int(start)]
    for _ in range(n - 1):
        out.append(int(inv[out[-1]]))
    return out
