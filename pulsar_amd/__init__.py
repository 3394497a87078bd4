"""pulsar_amd - MI355X (gfx950) quantized expert-matvec / routed-MoE library.

The product is libpulsar_moe.so (HIP kernels behind the C ABI in
include/pulsar_moe.h). This package builds it (`build`), binds it with the
reference's wrapper names (`kernels`), and carries the format table
(`formats`) and the seeded synthetic inputs of the benchmark configurations
(`synth`).
"""
from . import formats  # noqa: F401

__all__ = ["formats", "kernels", "synth", "build"]
