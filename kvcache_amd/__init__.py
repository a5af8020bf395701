"""kvcache_amd -- MI355X (gfx950) paged decode attention for continuously
re-batched ragged sequences: a drop-in for the decode hot path of
kimxinw/kvcache.

Layers:
  include/kvc_abi.h      C ABI of libkvcache_amd.so (HIP kernels for gfx950)
  include/kvc/*.h        C++ API with the reference's names (BlockAllocator,
                         KVCacheManager, ModelRunner, Engine, run_static, launch_*)
  kvcache_amd.ops        Python mirror of the reference's launch_* functions
  kvcache_amd.engine     Python handles over the C++ Engine / run_static
  kvcache_amd.workloads  reference and BASELINE workload generators
"""
from ._native import KVC_F16, KVC_F32, KvcError, LIB_PATH, lib  # noqa: F401

__version__ = "0.1.0"
