"""bsscl-gbm on MI355X: the reference's binary histogram-GBM estimator
(src/bsscl_gbm/__init__.py:5-9 exports HybridHistGBMNumbaV1_0_1) backed by
hand-written HIP kernels for gfx950."""

from .estimator import HybridHistGBMNumbaV1_0_1

__version__ = "1.0.1"
__all__ = ["HybridHistGBMNumbaV1_0_1"]
