"""MI355X (gfx950) palette-weight GEMM for parakeet.wgsl's FastConformer path.

Native code: lib/libpk_palette.so (HIP kernels + C ABI, include/pk_palette.h)
and lib/pk_napi.node (Node N-API addon). Python modules:
  palette_abi  ctypes binding of the C ABI (tests, benchmark)
  workloads    seeded synthetic inputs of the benchmark configurations
  build        compiles the native libraries in-tree
"""
__version__ = "0.1.0"
