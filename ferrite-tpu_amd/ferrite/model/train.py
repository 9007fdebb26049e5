"""Training loop for the GPT of :mod:`ferrite.model.gpt` on one MI355X, with a
hand-written AdamW.

Reference: src/ferrite/model/train.py. Same ``TrainConfig``, optimiser
(global-norm clipping, bias-corrected AdamW, decoupled weight decay on tensors
with ndim >= 2 only, linear warmup then cosine decay to 10% of the peak rate),
results dictionary, ``.npz`` checkpoint layout and command line.

Device placement: one process drives one GPU. The reference shards the batch
over a 1-D data mesh and lets XLA insert the gradient all-reduce
(train.py:80-99); this build trains on a single device, and a multi-GPU run
would add one all-reduce of the gradient list per step between the backward and
``adamw_update``. The optimiser runs on the fused HIP kernel
(``optimizer="fused"``, csrc/optim.hip: one pass over g, p, m, v per step) or
as torch multi-tensor (``_foreach``) ops (``optimizer="foreach"``, also on CPU);
both compute in f32, and with bf16 parameters the moments stay f32 and each
update is rounded once into the parameter.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import time
from typing import Any

import numpy as np
import torch

from ferrite import platform
from ferrite.graphs import capture_window
from ferrite.model import data as data_lib
from ferrite.model.gpt import GPTConfig, flops_per_token, init_params, leaves, loss_fn, named_leaves, param_count, unflatten


@dataclasses.dataclass(frozen=True)
class TrainConfig:
    """Run settings (train.py:29-41)."""

    steps: int = 200
    batch: int = 64
    lr: float = 6e-4
    warmup: int = 20
    weight_decay: float = 0.1
    clip: float = 1.0
    seed: int = 0
    log_every: int = 10
    data: str = "tinyshakespeare"
    out: str | None = None
    save_params: str | None = None
    optimizer: str = "fused"  # "fused" (HIP kernel) | "foreach" (torch multi-tensor ops)

    def __post_init__(self):
        if self.optimizer not in ("fused", "foreach"):
            raise ValueError(f"optimizer must be 'fused' or 'foreach', got {self.optimizer!r}")


def default_device() -> torch.device:
    return torch.device("cuda:0") if platform.is_rocm() else torch.device("cpu")


def _dtype_name(dt: torch.dtype) -> str:
    return str(dt).replace("torch.", "")


# ---------------------------------------------------------------- optimiser


def adamw_init(params) -> dict:
    """Zero first and second moments (f32) and a step counter (train.py:47-49)."""

    def zeros(t):
        return torch.zeros_like(t, dtype=torch.float32)

    m = unflatten(params, [zeros(t) for t in leaves(params)])
    v = unflatten(params, [zeros(t) for t in leaves(params)])
    return {"m": m, "v": v, "step": 0}


def lr_at(step: int, cfg: TrainConfig) -> float:
    """Linear warmup to ``cfg.lr``, then cosine decay to 10% of it (train.py:52-56)."""
    if step < cfg.warmup:
        return cfg.lr * (step + 1) / max(1, cfg.warmup)
    progress = min(max((step - cfg.warmup) / max(1, cfg.steps - cfg.warmup), 0.0), 1.0)
    return 0.1 * cfg.lr + 0.9 * cfg.lr * 0.5 * (1 + math.cos(math.pi * progress))


@torch.no_grad()
def adamw_update(params, grads, state, cfg: TrainConfig, b1: float = 0.9, b2: float = 0.95, eps: float = 1e-8):
    """One AdamW step (train.py:59-74), in place on ``params`` and ``state``.

    Gradients are clipped to a global f32 norm of ``cfg.clip`` (the f32 gradient
    tensors are scaled in place). Returns ``(params, state, gnorm)`` with ``gnorm``
    the pre-clip norm as a 0-d device tensor, so the step needs no host sync."""
    step = state["step"] + 1
    lr = lr_at(step, cfg)
    if cfg.optimizer == "fused":
        from ferrite.kernels.adamw import fused_adamw_

        p = leaves(params)
        gnorm = fused_adamw_(p, leaves(grads), leaves(state["m"]), leaves(state["v"]), [t.ndim >= 2 for t in p],
                             lr=lr, beta1=b1, beta2=b2, eps=eps, weight_decay=cfg.weight_decay,
                             max_grad_norm=cfg.clip, step=step)
        return params, {"m": state["m"], "v": state["v"], "step": step}, gnorm
    p = leaves(params)
    g = [t.float() for t in leaves(grads)]
    m = leaves(state["m"])
    v = leaves(state["v"])
    gnorm = torch.linalg.vector_norm(torch.stack(torch._foreach_norm(g)))
    torch._foreach_mul_(g, torch.clamp(cfg.clip / (gnorm + 1e-6), max=1.0))
    torch._foreach_mul_(m, b1)
    torch._foreach_add_(m, g, alpha=1 - b1)
    torch._foreach_mul_(v, b2)
    torch._foreach_addcmul_(v, g, g, value=1 - b2)
    bc1, bc2 = 1 - b1**step, 1 - b2**step
    denom = torch._foreach_div(v, bc2)
    torch._foreach_sqrt_(denom)
    torch._foreach_add_(denom, eps)
    upd = torch._foreach_div(m, bc1)
    torch._foreach_div_(upd, denom)
    pf = [t.float() for t in p]
    decayed = [i for i, t in enumerate(p) if t.ndim >= 2]  # no decay on norm gains
    if cfg.weight_decay and decayed:
        torch._foreach_add_([upd[i] for i in decayed], [pf[i] for i in decayed], alpha=cfg.weight_decay)
    torch._foreach_add_(pf, upd, alpha=-lr)
    for t, tf in zip(p, pf):
        if t is not tf:
            t.copy_(tf)
    return params, {"m": state["m"], "v": state["v"], "step": step}, gnorm


# ---------------------------------------------------------------- training


def value_and_grad(params, x, y, cfg: GPTConfig):
    """Loss and the gradient tree of ``loss_fn`` w.r.t. every parameter."""
    ps = leaves(params)
    for t in ps:
        if not t.requires_grad:
            t.requires_grad_(True)
    loss = loss_fn(params, x, y, cfg)
    grads = torch.autograd.grad(loss, ps)
    return loss.detach(), unflatten(params, list(grads))


def build_train_step(model_cfg: GPTConfig, train_cfg: TrainConfig, *, graph: bool = False):
    """``step(params, opt, x, y) -> (params, opt, loss, gnorm)``: forward, backward, AdamW
    (train.py:84-99, on one device).

    ``graph=True`` returns a :class:`GraphedTrainStep`: the same step captured once into a HIP
    graph and replayed, which removes the host's per-kernel launch cost (the role ``jax.jit``
    plays for the reference)."""
    if graph:
        return GraphedTrainStep(model_cfg, train_cfg)

    def step(params, opt, x, y):
        loss, grads = value_and_grad(params, x, y, model_cfg)
        params, opt, gnorm = adamw_update(params, grads, opt, train_cfg)
        return params, opt, loss, gnorm

    return step


class GraphedTrainStep:
    """The training step captured into a HIP graph and replayed (fused AdamW only).

    The first ``warmup`` calls run eagerly on a side stream (library handles, the autograd
    engine and the allocator settle there). The next call captures forward, backward and the
    AdamW update into a graph and replays it; later calls only replay. Everything the graph
    touches has a fixed address: the parameter and moment tensors, static token buffers the
    inputs are copied into, the loss and gradient-norm outputs, and a device vector holding
    the step's learning rate and bias corrections, refreshed before each replay (the update
    kernel reads them from memory, so the replayed arguments can stay fixed). Parameters and
    moments are updated in place, so ``params`` and ``opt`` must be the same trees on every call.
    The returned loss of a replayed step is the graph's output tensor, overwritten by the next
    replay: read it (or clone it) before calling again.
    """

    def __init__(self, model_cfg: GPTConfig, train_cfg: TrainConfig, warmup: int = 2, b1: float = 0.9,
                 b2: float = 0.95, eps: float = 1e-8):
        if train_cfg.optimizer != "fused":
            raise ValueError("a graphed step needs optimizer='fused' (its update reads per-step values from memory)")
        self.model_cfg, self.train_cfg = model_cfg, train_cfg
        self.warmup, self.b1, self.b2, self.eps = warmup, b1, b2, eps
        self.graph = None
        self.calls = 0

    def _setup(self, params, opt, x, y):
        dev = x.device
        self.x, self.y = torch.empty_like(x), torch.empty_like(y)
        self.scalars = torch.zeros(3, dtype=torch.float32, device=dev)
        self.gnorm = torch.zeros((), dtype=torch.float32, device=dev)
        self.ps = leaves(params)
        for t in self.ps:
            t.requires_grad_(True)
        self.ms, self.vs = leaves(opt["m"]), leaves(opt["v"])
        self.decay = [t.ndim >= 2 for t in self.ps]
        from ferrite import _hip

        n = len(self.ps)
        self.ws = torch.empty(((_hip.lib().ferrite_hip_adamw_workspace(n) + 3) // 4,), dtype=torch.float32, device=dev)
        self.side = torch.cuda.Stream(device=dev)

    def _body(self):
        """One step on the static buffers; returns the loss tensor."""
        from ferrite.kernels.adamw import fused_adamw_

        loss = loss_fn(self.params, self.x, self.y, self.model_cfg)
        grads = torch.autograd.grad(loss, self.ps)
        fused_adamw_(self.ps, list(grads), self.ms, self.vs, self.decay, lr=0.0, beta1=self.b1, beta2=self.b2,
                     eps=self.eps, weight_decay=self.train_cfg.weight_decay, max_grad_norm=self.train_cfg.clip,
                     step=1, step_scalars=self.scalars, grad_norm=self.gnorm, workspace=self.ws)
        return loss.detach()

    def __call__(self, params, opt, x, y):
        if self.calls == 0:
            self.params = params
            self._setup(params, opt, x, y)
        step = opt["step"] + 1
        # per-step values as fill kernels on the stream (no host buffer to race with the GPU)
        self.scalars[0].fill_(lr_at(step, self.train_cfg))
        self.scalars[1].fill_(1.0 - self.b1**step)
        self.scalars[2].fill_(1.0 - self.b2**step)
        self.x.copy_(x, non_blocking=True)
        self.y.copy_(y, non_blocking=True)
        if self.calls < self.warmup:
            self.side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(self.side):
                loss = self._body()
            torch.cuda.current_stream().wait_stream(self.side)
        else:
            if self.graph is None:
                torch.cuda.synchronize()
                self.graph = torch.cuda.CUDAGraph()
                with capture_window(), torch.cuda.graph(self.graph):
                    self.loss = self._body()
            self.graph.replay()
            loss = self.loss
        self.calls += 1
        return params, {"m": opt["m"], "v": opt["v"], "step": step}, loss, self.gnorm

    def close(self) -> None:
        """Destroy the captured graph once the device has finished with it. A later call starts
        over (warm-up, capture). Also called on leaving a ``with`` block."""
        if self.graph is not None:
            torch.cuda.synchronize()
            self.graph.reset()
            self.graph = None
            self.loss = None
        self.calls = 0

    def __enter__(self) -> "GraphedTrainStep":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def train(model_cfg: GPTConfig, train_cfg: TrainConfig, *, verbose: bool = True, device=None,
          graph: bool = False) -> dict[str, Any]:
    """Train for ``train_cfg.steps`` steps and return the results dictionary (train.py:102-177).
    ``graph=True`` replays the step from a captured HIP graph (see :class:`GraphedTrainStep`)."""
    device = torch.device(device) if device is not None else default_device()
    corpus = data_lib.load(train_cfg.data)
    train_data, _ = data_lib.split(corpus)
    rng = np.random.default_rng(train_cfg.seed)

    params = init_params(train_cfg.seed, model_cfg, device=device)
    n_params = param_count(params)
    n_nonembed = n_params - params["tok_emb"].numel() - params["pos_emb"].numel()
    opt = adamw_init(params)
    step_fn = build_train_step(model_cfg, train_cfg, graph=graph)

    def batch():
        x, y = data_lib.get_batch(rng, train_data, train_cfg.batch, model_cfg.seq_len)
        return torch.from_numpy(x).to(device), torch.from_numpy(y).to(device)

    tokens_per_step = train_cfg.batch * model_cfg.seq_len
    fpt = flops_per_token(model_cfg, n_nonembed)
    train_flops_per_step = 3 * fpt["total"] * tokens_per_step  # fwd + bwd (2x fwd)
    peaks = platform.peaks()
    peak_flops = peaks.bf16_flops if (peaks and device.type == "cuda") else None

    losses, step_times, gnorms = [], [], []
    first_step_s = float("nan")
    warm = min(5, train_cfg.steps // 4)
    for i in range(train_cfg.steps):
        x, y = batch()
        t = time.perf_counter()
        params, opt, loss, gnorm = step_fn(params, opt, x, y)
        loss = float(loss)  # waits for the whole step, optimiser included
        dt = time.perf_counter() - t
        losses.append(loss)
        gnorms.append(float(gnorm))
        if i == 0:
            first_step_s = dt
        if i >= warm:
            step_times.append(dt)
        if verbose and (i % train_cfg.log_every == 0 or i == train_cfg.steps - 1):
            print(f"step {i:5d} loss {loss:.4f} gnorm {gnorms[-1]:.3f} step {dt * 1e3:.1f} ms")

    med = float(np.median(step_times)) if step_times else float("nan")
    result = {
        "platform": platform.describe(),
        "model": {**dataclasses.asdict(model_cfg), "dtype": _dtype_name(model_cfg.dtype), "params": n_params, "params_nonembed": n_nonembed},
        "train": dataclasses.asdict(train_cfg),
        # No tracing compiler here: the first step's wall time (kernel library load and first launches).
        "compile_seconds": first_step_s,
        "step_ms_median": med * 1e3,
        "step_ms_min": float(np.min(step_times)) * 1e3 if step_times else float("nan"),
        "tokens_per_second": tokens_per_step / med if step_times else float("nan"),
        "train_flops_per_step_analytic": train_flops_per_step,
        "train_flops_per_step_xla_cost_analysis": None,
        "achieved_tflops": train_flops_per_step / med / 1e12 if step_times else float("nan"),
        "mfu": (train_flops_per_step / med / peak_flops) if (step_times and peak_flops) else None,
        "loss_first": losses[0],
        "loss_last": float(np.mean(losses[-10:])),
        "loss_curve": losses[:: max(1, len(losses) // 50)],
    }
    if train_cfg.out:
        os.makedirs(os.path.dirname(train_cfg.out) or ".", exist_ok=True)
        with open(train_cfg.out, "w") as f:
            json.dump(result, f, indent=2)
    if train_cfg.save_params:
        save_params(train_cfg.save_params, params)
    return result


def save_params(path: str, params) -> None:
    """``.npz`` with one f32 array per leaf, keyed "tok_emb", "layers/0/wqkv", ... (train.py:167-170)."""
    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    flat = {name: t.detach().float().cpu().numpy() for name, t in named_leaves(params)}
    np.savez(path, **flat)


def load_params(path: str, cfg: GPTConfig, *, device=None, dtype: torch.dtype = torch.float32) -> dict:
    """Inverse of :func:`save_params` (train.py:188-198)."""
    raw = np.load(path)
    params: dict = {"layers": [dict() for _ in range(cfg.n_layer)]}
    for k in raw.files:
        t = torch.from_numpy(raw[k]).to(device=device, dtype=dtype)
        parts = k.split("/")
        if parts[0] == "layers":
            params["layers"][int(parts[1])][parts[2]] = t
        else:
            params[parts[0]] = t
    return params


def main(argv=None):
    ap = argparse.ArgumentParser(description="Train the small transformer on the HIP kernels ('pallas') or plain torch ('xla').")
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--seq", type=int, default=256)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--d-model", type=int, default=512)
    ap.add_argument("--heads", type=int, default=4)
    ap.add_argument("--d-ff", type=int, default=2048)
    ap.add_argument("--attention", choices=["pallas", "xla"], default="pallas")
    ap.add_argument("--norm", choices=["pallas", "xla"], default="pallas")
    ap.add_argument("--linear", choices=["pallas", "xla"], default="xla")
    ap.add_argument("--loss", choices=["pallas", "xla"], default="pallas",
                    help="tied head + cross-entropy on the HIP loss kernels or torch's cross_entropy")
    ap.add_argument("--dtype", choices=["bfloat16", "float32"], default="bfloat16")
    ap.add_argument("--lr", type=float, default=6e-4)
    ap.add_argument("--data", choices=["tinyshakespeare", "synthetic"], default="tinyshakespeare")
    ap.add_argument("--out", default=None, help="results JSON path")
    ap.add_argument("--save-params", default=None, help=".npz checkpoint path")
    ap.add_argument("--optimizer", choices=["fused", "foreach"], default=None,
                    help="AdamW on the fused HIP kernel (default on a GPU) or torch multi-tensor ops (default on CPU)")
    ap.add_argument("--graph", action="store_true", help="replay the step from a captured HIP graph")
    a = ap.parse_args(argv)
    dtype = {"bfloat16": torch.bfloat16, "float32": torch.float32}[a.dtype]
    mcfg = GPTConfig(seq_len=a.seq, d_model=a.d_model, n_head=a.heads, n_layer=a.layers, d_ff=a.d_ff, attention=a.attention, norm=a.norm, linear=a.linear, loss=a.loss, dtype=dtype)
    optimizer = a.optimizer or ("fused" if platform.is_rocm() else "foreach")
    tcfg = TrainConfig(steps=a.steps, batch=a.batch, lr=a.lr, data=a.data, out=a.out, save_params=a.save_params,
                       optimizer=optimizer)
    with platform.interpret_mode():
        res = train(mcfg, tcfg, graph=a.graph)
    print(json.dumps({k: v for k, v in res.items() if k != "loss_curve"}, indent=2, default=str))


if __name__ == "__main__":
    main()
