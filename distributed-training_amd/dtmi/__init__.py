"""dtmi: dtrain's backward / gradient / optimizer path on the AMD Instinct MI355X.

The public modules mirror dtrain's (siddhaantxsingh/DISTRIBUTED-TRAINING):
`dtmi.autograd` (Tensor, backward, grad-ready hooks, ops), `dtmi.nn` (GPT),
`dtmi.optim` (AdamW over flat device buffers, clip_scale), `dtmi.ddp` (DDP
buckets with a fixed-order on-device average of simulated replicas) and
`dtmi.zero` (ZeRO-1 shard slicing). Arithmetic runs in hand-written gfx950
kernels of libdtmi.so, bound with ctypes (`dtmi._lib`); there is no CPU path.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
