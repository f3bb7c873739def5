"""ctypes mirror of the MI355X MoE library's C ABI (``include/*.h``).

The reference's callers reach its kernels through ``#[repr(C)]`` call structures
(``crates/ops/src/moe/*.rs``) and its Python kernel checks through ctypes mirrors of
the same structures (``tests/python/kernels/moe/test_moe_sort.py:56-84``); this
package is that mirror for the HIP library. It holds no fallback: loading fails
loudly when the shared object has not been built.
"""

from .abi import (  # noqa: F401
    DTYPE,
    GatherCall,
    GatherFp8Call,
    GemmCall,
    LayerCall,
    LayerViews,
    QuantizeFp8Call,
    MxStageScalesCall,
    QuantizeMxfp8Call,
    GatherMxCall,
    RouteMxCall,
    RouteCall,
    RouteFp8Call,
    SortCall,
    UnpermuteCall,
    LAYOUT_EXPANDED,
    LAYOUT_PERMUTED,
    library,
    library_path,
    max_tiles,
)
