"""MI355X (gfx950) quantized GGML_OP_MUL_MAT for CrispEmbed.

The product is native: libmq.so (HIP kernels + the C ABI of include/mq.h) and
libggml-mi355.so (a ggml backend on top of it, include/ggml-mi355.h).  This
Python package only loads those libraries for tests and benchmarks; there is no
Python compute path and no fallback -- if the library is missing, loading fails.
"""
from .mq import lib, MQError, TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_K  # noqa: F401
from .mq import Q8_0_X86, Q8_0_NEON, Q8_0_REF, PATH_AUTO, PATH_GEMV, PATH_GEMM  # noqa: F401
