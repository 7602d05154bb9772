"""Fused AdamW on flat parameter shards (one kernel pass per shard).

Replaces ``torch.optim.Adam(fused=True)`` as the reference builds it for each
FSDP module's flat shard (zorse_utils/pipeline.py:150-181) and steps it from
the reduce-grad callback (utils/patch.py:76-154).  The grad cast of
utils/patch.py:115-119 (reduce dtype -> fp32) is folded into the kernel: the
gradient is read in whatever float dtype it has.

Mixed precision: when a parameter is bf16 / fp16 (the compute copy the layer
runs on), the optimizer keeps an fp32 master copy in its state, updates the
master, m and v, and writes the rounded parameter back -- all in the same
pass.  With an fp32 parameter the update is in place.

``weight_decay`` is decoupled (AdamW); ``FusedAdam`` is the same optimizer
with weight decay fixed at 0, which is exactly ``torch.optim.Adam`` with its
defaults -- the reference's optimizer.
"""
from __future__ import annotations

import torch

from . import kernels as K


class FusedAdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        if lr < 0 or eps < 0 or weight_decay < 0:
            raise ValueError("lr, eps and weight_decay must be non-negative")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"invalid betas {betas}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps,
                                      weight_decay=weight_decay))
        self._step_hooks = {}   # param -> [callable(param)]

    def add_step_hook(self, p: torch.Tensor, fn) -> None:
        """``fn(p)`` runs after every step of ``p`` (after its version bump)."""
        self._step_hooks.setdefault(p, []).append(fn)

    def _init_state(self, p: torch.Tensor) -> dict:
        st = self.state[p]
        if not st:
            st["step"] = 0
            st["exp_avg"] = torch.zeros(p.numel(), device=p.device, dtype=torch.float32)
            st["exp_avg_sq"] = torch.zeros(p.numel(), device=p.device, dtype=torch.float32)
            if p.dtype != torch.float32:
                st["master"] = p.detach().reshape(-1).to(torch.float32)
        return st

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    self._step_one(group, p)
        return loss

    @torch.no_grad()
    def step_param(self, p: torch.Tensor) -> None:
        """Step ``p`` alone (the other parameters of this optimizer are left
        as they are, whatever their gradients): the per-parameter step of an
        optimizer-in-backward hook, which fires once per parameter as its
        gradient completes.  No-op when ``p.grad`` is None."""
        for group in self.param_groups:
            for q in group["params"]:
                if q is p:
                    if p.grad is not None:
                        self._step_one(group, p)
                    return
        raise ValueError("step_param: the tensor is not a parameter of this optimizer")

    def _step_one(self, group: dict, p: torch.Tensor) -> None:
        b1, b2 = group["betas"]
        if p.grad.is_sparse:
            raise RuntimeError("FusedAdamW does not support sparse gradients")
        if not p.is_contiguous() or not p.grad.is_contiguous():
            raise ValueError("FusedAdamW needs contiguous parameters and gradients")
        st = self._init_state(p)
        if st["exp_avg"].device != p.device:
            for k in ("exp_avg", "exp_avg_sq", "master"):
                if k in st:
                    st[k] = st[k].to(p.device)
        st["step"] += 1
        master = st.get("master")
        hyper = dict(lr=group["lr"], beta1=b1, beta2=b2, eps=group["eps"],
                     weight_decay=group["weight_decay"], step=st["step"])
        K.adamw_step(master if master is not None else p.view(-1),
                     p.grad.view(-1), st["exp_avg"], st["exp_avg_sq"],
                     lowp_out=p.view(-1) if master is not None else None, **hyper)
        # the kernel wrote p through a raw pointer: advance its version
        # counter as an in-place torch op would, so caches keyed on it
        # (compute-dtype weight copies, attention caches) see the update
        torch.autograd.graph.increment_version(p)
        for fn in self._step_hooks.get(p, ()):
            fn(p)

    def master_param(self, p: torch.Tensor) -> torch.Tensor:
        """fp32 master of ``p`` (``p`` itself when it is fp32)."""
        st = self._init_state(p)
        return st.get("master", p.view(-1))


class FusedAdam(FusedAdamW):
    """torch.optim.Adam's defaults (lr 1e-3, betas (0.9, 0.999), eps 1e-8,
    no weight decay) -- the optimizer the reference builds per flat shard."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        if weight_decay != 0:
            raise ValueError("FusedAdam applies no weight decay; use FusedAdamW for "
                             "decoupled weight decay")
        super().__init__(params, lr=lr, betas=betas, eps=eps, weight_decay=0.0)
