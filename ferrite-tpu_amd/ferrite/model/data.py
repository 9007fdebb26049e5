"""Byte-level corpora for the training loop: a local TinyShakespeare file, or a
synthetic Markov corpus.

Reference: src/ferrite/model/data.py. The synthetic corpus draws from numpy's
``default_rng(seed)`` in the reference's order (transition table, first two
symbols, branch choices, noise mask, noise symbols), so a seed gives the same
bytes. This build never downloads: the machines it runs on have no network, so
``load_tinyshakespeare`` reads an existing file and ``load`` falls back to the
synthetic corpus, as the reference does when its download fails (data.py:37-43).
"""

from __future__ import annotations

import os

import numpy as np

FILENAME = "tinyshakespeare.txt"


def load_tinyshakespeare(root: str = "data") -> np.ndarray:
    """The corpus as uint8 bytes from ``root/tinyshakespeare.txt`` (data.py:13-20, without the download)."""
    path = os.path.join(root, FILENAME)
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not found (this build does not download corpora)")
    with open(path, "rb") as f:
        return np.frombuffer(f.read(), dtype=np.uint8)


def synthetic(n: int = 1_000_000, seed: int = 0) -> np.ndarray:
    """A learnable fake corpus (data.py:23-34): an order-2 Markov chain over 64 symbols.

    Each symbol is one of three successors of the previous two, chosen uniformly;
    5% of positions are replaced by a uniform symbol instead."""
    rng = np.random.default_rng(seed)
    table = rng.integers(0, 64, size=(64, 64, 3))
    start = rng.integers(0, 64, size=2)
    choice = rng.integers(0, 3, size=n)
    noisy = rng.random(n) < 0.05
    rnd = rng.integers(0, 64, size=n)
    # The chain is sequential; plain Python ints over flattened lists keep it fast.
    succ = table.reshape(-1).tolist()
    choice_l, noisy_l, rnd_l = choice.tolist(), noisy.tolist(), rnd.tolist()
    seq = [0] * n
    seq[: min(n, 2)] = start.tolist()[: min(n, 2)]
    for i in range(2, n):
        seq[i] = rnd_l[i] if noisy_l[i] else succ[(seq[i - 2] * 64 + seq[i - 1]) * 3 + choice_l[i]]
    return np.asarray(seq, dtype=np.uint8)


def load(name: str) -> np.ndarray:
    """'tinyshakespeare' (local file, else the synthetic fallback) or 'synthetic'."""
    if name == "tinyshakespeare":
        try:
            return load_tinyshakespeare()
        except Exception as e:
            print(f"[data] tinyshakespeare unavailable ({e}); using synthetic corpus")
    return synthetic()


def split(data: np.ndarray, frac: float = 0.9):
    n = int(len(data) * frac)
    return data[:n], data[n:]


def get_batch(rng: np.random.Generator, data: np.ndarray, batch: int, seq_len: int):
    """Random contiguous windows -> (inputs, targets) as int32 [batch, seq_len] (data.py:51-56)."""
    starts = rng.integers(0, len(data) - seq_len - 1, size=batch)
    idx = starts[:, None] + np.arange(seq_len + 1)[None, :]
    chunk = data[idx].astype(np.int32)
    return chunk[:, :-1], chunk[:, 1:]
