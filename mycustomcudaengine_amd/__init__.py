"""MI355X-native (gfx950) attention hot path of a paged-KV Llama-3.2-3B engine.

`mycustomcudaengine_amd.ops` is the `my_cuda_engine_cpp` op surface (HIP
kernels in libmce.so behind a C ABI); `mycustomcudaengine_amd.engine` holds the
block allocator, graph runner, weight loader and Llama wrapper that drive it.
"""

__version__ = "0.1.0"
