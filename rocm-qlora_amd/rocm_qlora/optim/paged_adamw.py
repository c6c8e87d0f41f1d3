"""PagedAdamW on one fused HIP launch per step (optim/paged_adamw.py:15-176 of
the reference).

The reference keeps each parameter's exp_avg / exp_avg_sq in CPU pinned
memory and, per parameter and step, copies both to the GPU, runs nine torch
ops and copies them back (paged_adamw.py:67-127).  Here the states of all
parameters live in two flat fp32 buffers (each tensor's slice padded to a
whole number of 2048-element chunks; state['exp_avg'] / ['exp_avg_sq'] are
views of them, shaped like the parameter), and a step is one
`rq_adamw_step` launch over every parameter that has a gradient, with the
reference's update rule and order of operations (see include/rocm_qlora_amd.h).

offload_states=True (the default, the reference's memory behaviour): the
flat buffers are pinned host memory; a step streams them through two device
pages of page_size_mb each (copy in, update, copy out, page after page on
the current stream) and synchronizes at its end, as the reference does.
offload_states=False keeps the states in device memory (no copies, no
synchronization): on a GPU with HBM to spare, the faster choice.

Parameters must be contiguous and on one GPU; the step raises otherwise
(there is no CPU update path).
"""
from __future__ import annotations

from typing import Any, Dict, Iterable, List, Tuple

import numpy as np
import torch
from torch.optim import Optimizer

from rocm_qlora import _native as nat
from rocm_qlora._device import on

ADAMW_CHUNK = 2048  # RQ_ADAMW_CHUNK

# rq_adamw_tensor (72 bytes)
_TABLE = np.dtype([
    ("param", "<u8"), ("grad", "<u8"), ("numel", "<i8"), ("state_offset", "<i8"),
    ("dtype", "<i4"), ("apply_decay", "<i4"),
    ("decay", "<f4"), ("beta1", "<f4"), ("one_minus_beta1", "<f4"), ("beta2", "<f4"),
    ("one_minus_beta2", "<f4"), ("inv_bias_correction2_sqrt", "<f4"), ("eps", "<f4"), ("neg_step_size", "<f4"),
])
assert _TABLE.itemsize == 72


def _chunks(n: int) -> int:
    return -(-n // ADAMW_CHUNK)


class PagedAdamW(Optimizer):
    """AdamW (decoupled weight decay) whose step is one fused HIP launch."""

    def __init__(self, params: Iterable[torch.Tensor], lr: float = 2e-4, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 0.01, page_size_mb: int = 256,
                 offload_states: bool = True):
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if page_size_mb < 1:
            raise ValueError(f"Invalid page_size_mb: {page_size_mb}")
        self.page_size_mb = int(page_size_mb)
        self.offload_states = bool(offload_states)
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))
        self._build_layout()

    # ------------------------------------------------------------ layout
    def _params(self) -> List[torch.Tensor]:
        return [p for g in self.param_groups for p in g["params"]]

    def _build_layout(self) -> None:
        """Assign each parameter its chunk-aligned slice of the flat state
        buffers and point its state at it (keeping values already held)."""
        params = self._params()
        offsets, total = {}, 0
        for p in params:
            offsets[p] = total
            total += _chunks(p.numel()) * ADAMW_CHUNK
        total = max(total, ADAMW_CHUNK)
        devs = {p.device for p in params if p.device.type == "cuda"}
        self._device = next(iter(devs)) if len(devs) == 1 else None
        if self.offload_states or self._device is None:
            pin = torch.cuda.is_available()
            m = torch.zeros(total, dtype=torch.float32, pin_memory=pin)
            v = torch.zeros(total, dtype=torch.float32, pin_memory=pin)
        else:
            m = torch.zeros(total, dtype=torch.float32, device=self._device)
            v = torch.zeros(total, dtype=torch.float32, device=self._device)
        for p in params:
            st = self.state[p]
            o, n = offsets[p], p.numel()
            for key, flat in (("exp_avg", m), ("exp_avg_sq", v)):
                view = flat[o:o + n].view(p.shape)
                old = st.get(key)
                if old is not None:
                    view.copy_(old.detach().reshape(p.shape).to(torch.float32))
                st[key] = view
            st.setdefault("step", 0)
            st["param_device"] = p.device
        self._offsets, self._total, self._m, self._v = offsets, total, m, v
        self._pages = None  # device page buffers (offload), made on first use
        self._dev_table = None
        self._build_static()

    def _build_static(self) -> None:
        """The per-tensor descriptor fields that do not change between steps."""
        plist, gidx = [], []
        for gi, group in enumerate(self.param_groups):
            for p in group["params"]:
                plist.append(p)
                gidx.append(gi)
        st = np.zeros(len(plist), dtype=_TABLE)
        st["param"] = [p.data_ptr() for p in plist]
        st["numel"] = [p.numel() for p in plist]
        st["state_offset"] = [self._offsets[p] for p in plist]
        st["dtype"] = [nat.dtype_code(p.dtype) if p.dtype in (torch.float32, torch.bfloat16, torch.float16) else -1
                       for p in plist]
        self._static, self._plist, self._gidx = st, plist, gidx
        self._contig = [p.is_contiguous() for p in plist]
        self._states = [self.state[p] for p in plist]
        self._views = [(t["exp_avg"], t["exp_avg_sq"]) for t in self._states]

    def add_param_group(self, param_group: Dict[str, Any]) -> None:
        super().add_param_group(param_group)
        if hasattr(self, "_offsets"):
            self._build_layout()

    def _layout_intact(self) -> bool:
        """The parameter list is the one laid out and every state still holds
        its views of the flat buffers (load_state_dict or a hand-made state
        replaces them)."""
        if len(self._plist) != sum(len(g["params"]) for g in self.param_groups):
            return False
        state = self.state
        for p, st, (m, v) in zip(self._plist, self._states, self._views):
            if state.get(p) is not st or st.get("exp_avg") is not m or st.get("exp_avg_sq") is not v:
                return False
        return True

    # ------------------------------------------------------------- step
    def _table(self, dev: torch.device) -> Tuple[np.ndarray, List[torch.Tensor], List[Tuple[int, int]]]:
        """This step's descriptors (tensors with a gradient, in state order),
        the gradients to keep alive until the launch, and their chunk spans.
        Advances the step count of each listed tensor."""
        plist = self._plist
        if [p.data_ptr() for p in plist] != self._static["param"].tolist():
            self._build_static()  # a parameter's storage was replaced
        grads = [p.grad for p in plist]
        live = [i for i, g in enumerate(grads) if g is not None]
        keep, gptr = [], []
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        for i in live:
            g, p = grads[i], plist[i]
            if g.layout is not torch.strided:
                raise RuntimeError("PagedAdamW does not support sparse gradients")
            if g.dtype is not p.dtype:
                raise RuntimeError(f"gradient dtype {g.dtype} differs from parameter dtype {p.dtype}")
            if not self._contig[i]:
                raise RuntimeError("PagedAdamW updates parameters in place: they must be contiguous")
            if g.get_device() != idx or p.get_device() != idx:
                raise RuntimeError(f"PagedAdamW: every parameter and gradient must be on {dev}")
            if not g.is_contiguous():
                g = g.contiguous()
            keep.append(g)
            gptr.append(g.data_ptr())
        if (self._static["dtype"][live] < 0).any():
            raise RuntimeError("PagedAdamW updates fp32, bf16 and fp16 parameters")
        rows = self._static[live]
        rows["grad"] = gptr
        # per (group, step) scalars, in the reference's double arithmetic
        cache, vals = {}, []
        groups = self.param_groups
        for i in live:
            st = self._states[i]
            st["step"] += 1
            key = (self._gidx[i], st["step"])
            v = cache.get(key)
            if v is None:
                grp = groups[key[0]]
                beta1, beta2 = grp["betas"]
                lr, wd, eps, t = grp["lr"], grp["weight_decay"], grp["eps"], key[1]
                bc1 = 1 - beta1 ** t                                      # paged_adamw.py:94-95
                bc2 = 1 - beta2 ** t
                # the division by bc2 ** 0.5 (paged_adamw.py:110) is a multiply
                # by its reciprocal, taken in double, in torch's GPU kernel
                v = cache[key] = (int(wd != 0), 1 - lr * wd, beta1, 1 - beta1, beta2, 1 - beta2,
                                  1.0 / bc2 ** 0.5, eps, -(lr / bc1))
            vals.append(v)
        if vals:
            cols = list(zip(*vals))
            rows["apply_decay"] = cols[0]
            for name, col in zip(("decay", "beta1", "one_minus_beta1", "beta2", "one_minus_beta2",
                                  "inv_bias_correction2_sqrt", "eps", "neg_step_size"), cols[1:]):
                rows[name] = np.asarray(col, dtype=np.float64)  # rounded to fp32 once, to nearest
        first = rows["state_offset"] // ADAMW_CHUNK
        spans = list(zip(first.tolist(), (first + (rows["numel"] + ADAMW_CHUNK - 1) // ADAMW_CHUNK).tolist()))
        return rows, keep, spans

    def _launch(self, table: np.ndarray, c0: int, c1: int, m: torch.Tensor, v: torch.Tensor) -> None:
        need = table.nbytes
        if self._dev_table is None or self._dev_table.numel() < need:
            self._dev_table = torch.empty(max(need, 4096), dtype=torch.uint8, device=self._device)
        nat.call("rq_adamw_step", table.ctypes.data, len(table), self._dev_table.data_ptr(), self._dev_table.numel(),
                 c0, c1, m.data_ptr(), v.data_ptr(), nat.stream_handle(self._device))

    @torch.no_grad()
    def step(self, closure=None):
        """One AdamW step of every parameter with a gradient
        (paged_adamw.py:67-127): one fused launch (per page of states when
        they are offloaded)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if not any(p.grad is not None for p in self._params()):
            return loss
        if self._device is None:
            raise RuntimeError("PagedAdamW steps on the GPU: all parameters must be on one GPU")
        if not self._layout_intact():
            self._build_layout()
        dev = self._device
        table, keep, spans = self._table(dev)
        with on(dev):
            if not self.offload_states:
                self._launch(table, 0, self._total // ADAMW_CHUNK, self._m, self._v)
            else:
                self._paged_step(table, spans)
                torch.cuda.current_stream(dev).synchronize()  # host states final, as the reference's sync
        del keep
        return loss

    def _paged_step(self, table: np.ndarray, spans: List[Tuple[int, int]]) -> None:
        page = max(1, (self.page_size_mb << 20) // (4 * ADAMW_CHUNK))  # chunks per page
        if self._pages is None or self._pages[0].numel() < page * ADAMW_CHUNK:
            n = min(page, self._total // ADAMW_CHUNK) * ADAMW_CHUNK
            self._pages = (torch.empty(n, dtype=torch.float32, device=self._device),
                           torch.empty(n, dtype=torch.float32, device=self._device))
        pm, pv = self._pages
        page = pm.numel() // ADAMW_CHUNK
        # fixed windows of `page` chunks; in each, the span of the chunks of
        # tensors updated this step
        windows: Dict[int, Tuple[int, int]] = {}
        for c_lo, c_hi in spans:
            for w in range(c_lo // page, (c_hi - 1) // page + 1) if c_hi > c_lo else ():
                a, b = max(c_lo, w * page), min(c_hi, (w + 1) * page)
                lo, hi = windows.get(w, (a, b))
                windows[w] = (min(lo, a), max(hi, b))
        for w in sorted(windows):
            c0, c1 = windows[w]
            lo, hi = c0 * ADAMW_CHUNK, c1 * ADAMW_CHUNK
            pm[:hi - lo].copy_(self._m[lo:hi], non_blocking=True)
            pv[:hi - lo].copy_(self._v[lo:hi], non_blocking=True)
            self._launch(table, c0, c1, pm, pv)
            self._m[lo:hi].copy_(pm[:hi - lo], non_blocking=True)
            self._v[lo:hi].copy_(pv[:hi - lo], non_blocking=True)

    # ----------------------------------------------------------- extras
    def get_memory_stats(self) -> Dict[str, Any]:
        """{cpu_pinned_mb, gpu_active_mb, num_params} (paged_adamw.py:129-151):
        state bytes held in pinned host memory and in device memory (the
        resident states, or the two pages of an offloaded step)."""
        state_bytes = sum(p.numel() for p in self._offsets) * 4 * 2
        gpu = 0
        if not self.offload_states and self._device is not None:
            gpu = state_bytes
        elif self._pages is not None:
            gpu = sum(t.numel() * 4 for t in self._pages)
        host = state_bytes if (self.offload_states or self._device is None) else 0
        return {"cpu_pinned_mb": host / (1024 * 1024), "gpu_active_mb": gpu / (1024 * 1024),
                "num_params": len(self._offsets)}

    def load_state_dict(self, state_dict: Dict[str, Any]) -> None:
        """Load, then put the states back into the flat buffers (pinned host
        or device, as configured) -- paged_adamw.py:161-176."""
        super().load_state_dict(state_dict)
        self._build_layout()
