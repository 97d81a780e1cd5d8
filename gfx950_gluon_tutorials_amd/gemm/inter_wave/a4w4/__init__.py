from .matmul_kernel import *  # noqa: F401,F403
from .matmul_kernel import matmul  # noqa: F401
