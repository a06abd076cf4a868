"""The drop-in slot (the role of the reference's kernel.py): KERNEL_TYPE + kernel_fn.

`python -m autokernel_amd.harness` imports this module when no --kernel is given. Point it at
another op by changing both lines, e.g. KERNEL_TYPE = "softmax" with
`from autokernel_amd.kernels.softmax import kernel_fn`.
"""
KERNEL_TYPE = "matmul"
from autokernel_amd.kernels.matmul import kernel_fn  # noqa: E402,F401
