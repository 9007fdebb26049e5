"""Greedy decoding with a static KV cache, replayed from captured HIP graphs.

Reference: src/ferrite/serving/engine.py. Same split between prefill and decode,
same cache layout, bucketing, API and statistics:

* Prompts are right-padded to one of a few **buckets**. The reference compiles
  each bucket's prefill ahead of time; here each bucket's prefill is captured
  once into a HIP graph, and serving replays it, so no launch at serving time
  depends on the Python model code.
* The KV cache is a fixed ``[layers, batch, heads, max_len, head_dim]`` buffer
  updated in place, and the decode step is one captured graph whatever the
  position (positions live in device memory).
* Prefill is compute-bound and runs the flash-attention kernel. Decode is
  memory-bound: the reference leaves it to XLA and names a decode-attention
  kernel as its next step; here ``decode_kernels="pallas"`` runs that kernel
  (csrc/decode.hip), which writes the new key/value rows and attends over the
  cache in one launch per layer.
* ``jax.export`` (engine.py:206-228) has no counterpart: a captured graph is the
  serialisation-free analogue, and it lives in the serving process.
"""

from __future__ import annotations

import dataclasses
import math
import time
from typing import Any

import numpy as np
import torch

from ferrite.graphs import capture_window
from ferrite.model.gpt import GPTConfig, _attention, _dot_f32, _linear, _merge_heads, _mlp, _norm, _split_heads


@dataclasses.dataclass(frozen=True)
class ServeConfig:
    """Serving settings (engine.py:35-40)."""

    batch: int = 1
    max_len: int = 512
    buckets: tuple[int, ...] = (64, 128, 256)
    prefill_kernels: str = "pallas"  # prefill's attention and norms: HIP kernels ("pallas") or torch ("xla")
    decode_kernels: str = "pallas"  # decode: HIP decode attention and norms ("pallas"), or torch math ("xla")
    graphs: bool = True  # capture prefill and decode as HIP graphs and replay them


def bucket_for(length: int, buckets: tuple[int, ...]) -> int:
    """The smallest bucket that holds ``length`` tokens (engine.py:43-47)."""
    for b in buckets:
        if length <= b:
            return b
    raise ValueError(f"no bucket holds a {length}-token prompt (buckets go up to {buckets[-1]})")


# The model, split into the prefill and decode passes.


def _block_prefill(layer, h, pending, cfg: GPTConfig):
    """Runs a block on a whole padded prompt. Returns the residual stream, the MLP output still to
    be added by the next norm, and the block's keys and values [B, H, S, hd] for the cache
    (engine.py:53-66)."""
    if pending is None:
        y = _norm(h, layer["ln1"], None, cfg)
    else:
        h, y = _norm(pending, layer["ln1"], h, cfg)
    q, k, v = _split_heads(_linear(y, layer["wqkv"], cfg), cfg)  # [B, H, S, hd]
    a = _linear(_merge_heads(_attention(q, k, v, cfg), cfg), layer["wo"], cfg)
    h, y2 = _norm(a, layer["ln2"], h, cfg)
    pending = _mlp(y2, layer, cfg)
    return h, pending, k, v


@torch.no_grad()
def prefill(params, tokens, lengths, cfg: GPTConfig, max_len: int, k_cache=None, v_cache=None):
    """Runs the model over right-padded prompts ``tokens`` [B, L] whose true lengths are
    ``lengths`` [B], and returns the logits of each prompt's last real token [B, V] with the
    two caches [layers, B, H, max_len, hd] (engine.py:69-86). Cache rows 0..L-1 receive the
    prompt's keys and values; rows past a prompt's length hold padding that decode masks out
    and overwrites as it goes. Caches passed in are filled in place."""
    b, s = tokens.shape
    if k_cache is None:
        shape = (cfg.n_layer, b, cfg.n_head, max_len, cfg.head_dim)
        k_cache = torch.zeros(shape, dtype=cfg.dtype, device=tokens.device)
        v_cache = torch.zeros(shape, dtype=cfg.dtype, device=tokens.device)
    h = (params["tok_emb"][tokens] + params["pos_emb"][:s]).to(cfg.dtype)
    pending = None
    for i, layer in enumerate(params["layers"]):
        h, pending, k, v = _block_prefill(layer, h, pending, cfg)
        k_cache[i, :, :, :s].copy_(k)
        v_cache[i, :, :, :s].copy_(v)
    _, y = _norm(pending, params["ln_f"], h, cfg)
    idx = (lengths.long() - 1).view(b, 1, 1).expand(b, 1, cfg.d_model)
    last = torch.gather(y, 1, idx)[:, 0]  # [B, d]
    logits = _dot_f32(last.contiguous(), params["tok_emb"].to(cfg.dtype).t())
    return logits, k_cache, v_cache


def _cache_attention(q, k_cache, v_cache, pos, scale):
    """Attention of one new query per sequence (q [B, H, hd]) over the cache rows up to and
    including its position pos [B], with f32 scores (engine.py:89-95)."""
    s = torch.einsum("bhd,bhkd->bhk", q.float(), k_cache.float()) * scale
    keys = torch.arange(k_cache.shape[2], device=q.device)[None, :]
    s = torch.where((keys <= pos.long()[:, None])[:, None, :], s, torch.full_like(s, -1e30))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bhk,bhkd->bhd", p, v_cache.float()).to(q.dtype)


def _write_cache(cache, new, pos):
    """Stores each sequence's new row (new [B, H, hd]) at its own position pos[b] of the cache
    [B, H, max_len, hd], in place (engine.py:98-104)."""
    idx = torch.arange(cache.shape[0], device=cache.device)
    cache[idx, :, pos.long()] = new.to(cache.dtype)


@torch.no_grad()
def decode_step(params, token, pos, k_cache, v_cache, cfg: GPTConfig):
    """Advances every sequence by one token: feeds ``token`` [B] at positions ``pos`` [B],
    writes their keys and values into the caches and returns the next logits [B, V]
    (engine.py:107-131). With ``cfg.attention == "pallas"`` the HIP decode-attention kernel does
    the cache write and the attention; otherwise torch restates the reference's XLA math."""
    b = token.shape[0]
    h = (params["tok_emb"][token] + params["pos_emb"][pos.long()]).to(cfg.dtype)  # [B, d]
    scale = 1.0 / math.sqrt(cfg.head_dim)
    pending = None
    for i, layer in enumerate(params["layers"]):
        if pending is None:
            y = _norm(h, layer["ln1"], None, cfg)
        else:
            h, y = _norm(pending, layer["ln1"], h, cfg)
        qkv = _linear(y, layer["wqkv"], cfg).reshape(b, 3, cfg.n_head, cfg.head_dim)
        q, k, v = (qkv[:, j].contiguous() for j in range(3))  # [B, H, hd]
        if cfg.attention == "pallas":
            from ferrite.kernels.decode_attention import decode_attention

            a = decode_attention(q, k, v, k_cache[i], v_cache[i], pos, scale=scale)
        else:
            _write_cache(k_cache[i], k, pos)
            _write_cache(v_cache[i], v, pos)
            a = _cache_attention(q, k_cache[i], v_cache[i], pos, scale)
        a = _linear(a.reshape(b, cfg.d_model), layer["wo"], cfg)
        h, y2 = _norm(a, layer["ln2"], h, cfg)
        pending = _mlp(y2, layer, cfg)
    _, y = _norm(pending, params["ln_f"], h, cfg)
    return _dot_f32(y, params["tok_emb"].to(cfg.dtype).t())


# The serving engine: captured prefill per bucket, one captured decode step.


class _Captured:
    """A function of fixed-address tensors, run eagerly once and then captured into a HIP graph."""

    def __init__(self, fn, graphs: bool):
        self.fn, self.graphs = fn, graphs
        self.graph = None
        self.out = None

    def __call__(self):
        if not self.graphs:
            return self.fn()
        if self.graph is None:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self.fn()  # warm-up: library handles, allocator, kernel attributes
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with capture_window(), torch.cuda.graph(self.graph):
                self.out = self.fn()
        self.graph.replay()
        return self.out

    def close(self) -> None:
        """Destroy the graph (after the device has finished any replay of it) and its output."""
        if self.graph is not None:
            torch.cuda.synchronize()
            self.graph.reset()
            self.graph = None
        self.out = None


class Engine:
    """Serves greedy generation from captured HIP graphs: one prefill graph per prompt bucket
    and one decode-step graph, all built when the engine is constructed (engine.py:137-203).
    Usable as a context manager; ``close()`` releases the graphs and ends the engine's use."""

    def __init__(self, params, model_cfg: GPTConfig, serve_cfg: ServeConfig, device=None):
        if max(serve_cfg.buckets) > model_cfg.seq_len or serve_cfg.max_len > model_cfg.seq_len:
            raise ValueError(f"the model's positional table has {model_cfg.seq_len} rows: buckets and max_len "
                             "cannot exceed it")
        if max(serve_cfg.buckets) > serve_cfg.max_len:
            raise ValueError("buckets must fit within max_len")
        self.params = params
        self.cfg = model_cfg
        self.serve = serve_cfg
        self.device = torch.device(device) if device is not None else params["tok_emb"].device
        use_graphs = serve_cfg.graphs and self.device.type == "cuda"
        if serve_cfg.prefill_kernels == "pallas":
            self.prefill_cfg = model_cfg
        else:
            self.prefill_cfg = model_cfg.replace(attention="xla", norm="xla")
        if serve_cfg.decode_kernels == "pallas":
            self.decode_cfg = model_cfg
        else:
            self.decode_cfg = model_cfg.replace(attention="xla", norm="xla", linear="xla")
        b, dev = serve_cfg.batch, self.device
        shape = (model_cfg.n_layer, b, model_cfg.n_head, serve_cfg.max_len, model_cfg.head_dim)
        self.k_cache = torch.zeros(shape, dtype=model_cfg.dtype, device=dev)
        self.v_cache = torch.zeros(shape, dtype=model_cfg.dtype, device=dev)
        self.lengths = torch.ones((b,), dtype=torch.int32, device=dev)
        self.token = torch.zeros((b,), dtype=torch.long, device=dev)
        self.pos = torch.zeros((b,), dtype=torch.int32, device=dev)
        self.compile_seconds: dict[str, float] = {}
        self._closed = False
        self._prefill: dict[int, Any] = {}
        self._tokens: dict[int, torch.Tensor] = {}
        # The captured functions hold the tensors they use, not the engine: no reference cycle,
        # so a dropped engine frees its graphs at once.
        p_, kc, vc, lens, tok, pos = self.params, self.k_cache, self.v_cache, self.lengths, self.token, self.pos
        pcfg, dcfg, max_len = self.prefill_cfg, self.decode_cfg, serve_cfg.max_len
        for bucket in serve_cfg.buckets:
            t0 = time.perf_counter()
            toks = torch.zeros((b, bucket), dtype=torch.long, device=dev)
            self._tokens[bucket] = toks

            def run(toks=toks):
                logits, _, _ = prefill(p_, toks, lens, pcfg, max_len, kc, vc)
                return logits

            self._prefill[bucket] = _Captured(run, use_graphs)
            self._prefill[bucket]()  # capture now, as the reference compiles ahead of time
            self.compile_seconds[f"prefill_{bucket}"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        self._decode = _Captured(lambda: decode_step(p_, tok, pos, kc, vc, dcfg), use_graphs)
        self._decode()
        self.compile_seconds["decode"] = time.perf_counter() - t0
        self.n_compiles = len(self.compile_seconds)
        self.k_cache.zero_()
        self.v_cache.zero_()

    # Lifetime.

    def close(self) -> None:
        """Releases the captured graphs (every prefill bucket and the decode step) at once; leaving
        a ``with`` block does the same. A closed engine refuses further prefill, decode and
        generate calls. Closing twice is harmless."""
        for cap in self._prefill.values():
            cap.close()
        self._decode.close()
        self._prefill.clear()
        self._closed = True

    def _check_open(self) -> None:
        if self._closed:
            raise RuntimeError("engine closed: its graphs were released by close(); build a new Engine to serve")

    def __enter__(self) -> "Engine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    # Serving.

    def prefill(self, prompts: list[list[int]]):
        """Pads the prompts on the right to the smallest bucket that holds them, replays that
        bucket's prefill graph and returns the greedy first token of each [B], the positions
        decode continues from (the prompt lengths) [B], and the two caches."""
        self._check_open()
        b = self.serve.batch
        if len(prompts) != b:
            raise ValueError(f"this engine serves {b} prompt(s) at a time; {len(prompts)} given")
        lengths = np.array([len(p) for p in prompts], np.int32)
        if lengths.min() < 1:
            raise ValueError("every prompt needs at least one token")
        bucket = bucket_for(int(lengths.max()), self.serve.buckets)
        tokens = np.zeros((b, bucket), np.int64)
        for i, p in enumerate(prompts):
            tokens[i, : len(p)] = p
        self._tokens[bucket].copy_(torch.from_numpy(tokens))
        self.lengths.copy_(torch.from_numpy(lengths))
        logits = self._prefill[bucket]()
        return torch.argmax(logits, dim=-1), self.lengths.clone(), self.k_cache, self.v_cache

    def decode(self, token, pos, kc=None, vc=None):
        """Replays the decode graph for ``token`` [B] at positions ``pos`` [B] and returns the
        greedy next token [B] and the two caches (``kc`` / ``vc`` are accepted for the
        reference's signature; the engine always uses its own caches)."""
        self._check_open()
        self.token.copy_(token)
        self.pos.copy_(pos)
        logits = self._decode()
        return torch.argmax(logits, dim=-1), self.k_cache, self.v_cache

    def generate(self, prompts: list[list[int]], max_new_tokens: int) -> tuple[np.ndarray, dict]:
        """Generates ``max_new_tokens`` tokens per prompt greedily. Returns them as an array
        [B, max_new_tokens] and a dict of timings: time to first token, median and p99
        inter-token latency, tokens per second, total seconds and the number of captures."""
        self._check_open()
        if max(len(p) for p in prompts) + max_new_tokens > self.serve.max_len:
            raise ValueError(f"the longest prompt plus {max_new_tokens} new tokens does not fit the "
                             f"{self.serve.max_len}-row cache")
        sync = torch.cuda.synchronize if self.device.type == "cuda" else (lambda: None)
        t0 = time.perf_counter()
        token, pos, _, _ = self.prefill(prompts)
        out = [token.cpu().numpy()]  # waits for the prefill
        ttft = time.perf_counter() - t0
        step_times = []
        for _ in range(max_new_tokens - 1):
            t = time.perf_counter()
            token, _, _ = self.decode(token, pos)
            out.append(token.cpu().numpy())
            step_times.append(time.perf_counter() - t)
            pos = pos + 1
        sync()
        total = time.perf_counter() - t0
        stats = {
            "ttft_ms": ttft * 1e3,
            "itl_ms_median": float(np.median(step_times)) * 1e3 if step_times else float("nan"),
            "itl_ms_p99": float(np.percentile(step_times, 99)) * 1e3 if step_times else float("nan"),
            "tokens_per_second": len(prompts) * max_new_tokens / total,
            "total_s": total,
            "n_compiles": self.n_compiles,
        }
        return np.stack(out, axis=1), stats


@torch.no_grad()
def reference_greedy(params, cfg: GPTConfig, prompt: list[int], max_new_tokens: int) -> np.ndarray:
    """Greedy decoding without a cache, as a check on the engine: every step runs the whole
    model over the prompt and the tokens so far (engine.py:231-242)."""
    from ferrite.model.gpt import forward

    dev = params["tok_emb"].device
    toks = list(prompt)
    out = []
    for _ in range(max_new_tokens):
        logits = forward(params, torch.tensor([toks], dtype=torch.long, device=dev), cfg)
        nxt = int(torch.argmax(logits[0, -1]))
        out.append(nxt)
        toks.append(nxt)
    return np.array(out)
