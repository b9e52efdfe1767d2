"""MI355X-native resident decode epoch (HIP library + Python host side).

The hot path lives in ``csrc/`` (hand-written gfx950 kernels and the C-ABI of
``include/resident_epoch.h``, built into ``lib/libresident_epoch.so``); the
Python modules mirror the reference's ``vllm_ascend_resident_epoch`` host
interface on top of it.
"""

__all__ = ["runtime"]
