"""SPK package toolchain: graph IR, fusion passes, arena planner, KernelSpec
selection, the package writer, model generators and INT8 quantization."""

from .graph import Graph  # noqa: F401
from .writer import Protection, QuantParam, write_spk  # noqa: F401
