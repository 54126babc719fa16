"""AdamW on gfx950: the optimizer the reference builds (training/engine.py:10-16,
torch.optim.AdamW(groups, ..., foreach=False, fused=True)) with its step in the HIP kernel
ct_adamw_step.

`FusedAdamW` takes torch.optim.AdamW's arguments and keeps its state layout (per
parameter: a fp32 `step` tensor on the parameter's device, `exp_avg` and `exp_avg_sq` in
the parameter's dtype), so checkpoints written for the reference's fused optimizer load
unchanged (checkpointing/io.py:205-222 checks exactly these keys, shapes and dtypes).
Each step is one launch per parameter group and dtype: the step counters are incremented
and every tensor is updated from a device-side table of (param, grad, exp_avg,
exp_avg_sq, step, numel) rows and a list of fixed-size chunks. Parameters must live on
the HIP device in fp32 or bf16 with dense gradients of the same dtype; amsgrad is not
supported (the reference does not use it).
"""

import torch

from .kernels import _native

_CHUNK = 1 << 16  # elements per workgroup


class FusedAdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, amsgrad=False, *,
                 maximize=False, foreach=None, capturable=False, differentiable=False, fused=True):
        if not 0.0 <= float(lr):
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameters: {betas}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if amsgrad:
            raise NotImplementedError("FusedAdamW: amsgrad is not supported")
        if differentiable:
            raise NotImplementedError("FusedAdamW: differentiable updates are not supported")
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, amsgrad=False, maximize=maximize,
                        foreach=foreach, capturable=capturable, differentiable=False, fused=True)
        super().__init__(params, defaults)
        self._tables = {}

    def _state_of(self, p):
        state = self.state[p]
        if not state:
            state["step"] = torch.zeros((), dtype=torch.float32, device=p.device)
            state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
            state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
        return state

    def _table(self, slot, rows, device):
        """Device copies of the tensor table and the chunk list of one (group, device,
        dtype) slot, reused while the same storages take part in the step."""
        key = tuple(rows)
        cached = self._tables.get(slot)
        if cached is not None and cached[0] == key:
            return cached[1], cached[2]
        table = torch.tensor([list(r) for r in rows], dtype=torch.int64).reshape(-1, 6)
        chunks = [(index, start) for index, r in enumerate(rows) for start in range(0, r[5], _CHUNK)]
        chunk_list = torch.tensor(chunks, dtype=torch.int64).reshape(-1, 2)
        # Pinned host copies go up asynchronously on the current stream (no host wait); the
        # pinned allocator keeps their blocks until the copies are done.
        entry = (key, table.pin_memory().to(device, non_blocking=True),
                 chunk_list.pin_memory().to(device, non_blocking=True))
        self._tables[slot] = entry
        return entry[1], entry[2]

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = _native.library()
        for index, group in enumerate(self.param_groups):
            beta1, beta2 = group["betas"]
            buckets = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("FusedAdamW does not support sparse gradients")
                if not p.is_cuda or p.dtype not in (torch.float32, torch.bfloat16):
                    raise NotImplementedError("FusedAdamW: parameters must be fp32 or bf16 device tensors")
                if p.grad.dtype != p.dtype or not p.is_contiguous() or not p.grad.is_contiguous():
                    raise NotImplementedError("FusedAdamW: contiguous gradients of the parameter's dtype required")
                state = self._state_of(p)
                buckets.setdefault((p.device, p.dtype), []).append((p, state))
            for (device, dtype), members in buckets.items():
                rows = [(p.data_ptr(), p.grad.data_ptr(), s["exp_avg"].data_ptr(), s["exp_avg_sq"].data_ptr(),
                         s["step"].data_ptr(), p.numel()) for p, s in members if p.numel()]
                if not rows:
                    for _, s in members:
                        s["step"] += 1
                    continue
                for p, s in members:
                    if not p.numel():
                        s["step"] += 1
                table, chunks = self._table((index, device, dtype), rows, device)
                with torch.cuda.device(device):
                    status = lib.ct_adamw_step(
                        _native.ptr(table), len(rows), _native.ptr(chunks), len(chunks), _CHUNK,
                        _native.dtype_code(dtype), float(group["lr"]), float(beta1), float(beta2),
                        float(group["eps"]), float(group["weight_decay"]), int(bool(group["maximize"])), 1,
                        _native.stream_of(members[0][0]))
                _native.check(status, "ct_adamw_step")
        return loss
