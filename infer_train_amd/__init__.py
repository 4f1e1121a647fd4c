"""infer_train_amd -- MI355X (gfx950) KV-cache hot path for InferTrain.

Native library: infer_train_amd/libit_kv.so (C ABI in include/it_kv.h),
hand-written HIP kernels for slot-mapped append, block-table gather, evict,
Q8_0 / Q4_0 / Q4_1 / Q5_0 / Q5_1 quantise-append, paged split-K flash-decode and MFMA chunked prefill,
plus the host-side allocator and slot manager.  Python mirrors the
reference crate's API surface (memory::paged, batcher, Backend).
"""
from ._lib import (BF16, BLOCK_Q4_0_BYTES, BLOCK_Q4_1_BYTES, BLOCK_Q5_0_BYTES, BLOCK_Q5_1_BYTES, BLOCK_Q8_0_BYTES,
                   BLOCK_SIZE, F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, QK4_0, QK4_1, QK5_0, QK5_1, QK8_0, QUANT_TYPES,
                   DeviceError, InvalidInput, NotImplementedOp, OpError, lib)
from .memory import BlockPool
from .batcher import ContinuousBatcher, KvManager, StepPlan

__all__ = ["BF16", "F16", "F32", "Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q8_0", "QK4_0", "QK4_1", "QK5_0", "QK5_1", "QK8_0",
           "QUANT_TYPES", "BLOCK_SIZE", "BLOCK_Q4_0_BYTES", "BLOCK_Q4_1_BYTES", "BLOCK_Q5_0_BYTES", "BLOCK_Q5_1_BYTES",
           "BLOCK_Q8_0_BYTES", "OpError", "InvalidInput",
           "NotImplementedOp", "DeviceError", "lib", "BlockPool", "KvManager", "ContinuousBatcher", "StepPlan"]
