"""Drop-in module name of the reference's extension (setup.py:22-26,
csrc/bindings.cpp:22-29): `import my_cuda_engine_cpp` gets the six ops,
backed by the gfx950 kernels in mycustomcudaengine_amd/libmce.so."""
from mycustomcudaengine_amd.ops import (  # noqa: F401
    paged_attention_decode,
    paged_kv_store,
    prefill_attention,
    rmsnorm,
    rope_inplace,
    swiglu,
)
