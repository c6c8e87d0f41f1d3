"""Optimizers (optim/__init__.py of the reference): PagedAdamW, whose step is
one fused HIP launch over all parameters."""
from rocm_qlora.optim.paged_adamw import PagedAdamW

__all__ = ["PagedAdamW"]
