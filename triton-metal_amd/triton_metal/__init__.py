"""triton_metal (MI355X): ctypes shim over libtritonmetal.so, the tm_* C ABI.

The package keeps the reference's module layout (python/triton_metal/_core.py,
buffer.py) so that callers written against it import the same names.  All work
(kernel planning, launches, allocation, copies) happens inside the native
library; this package marshals arguments and adds the reference's host-side
drivers for the dense hot path (ops.py).
"""

__version__ = "0.0.1"
