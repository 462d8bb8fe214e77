"""joule_amd: the MoE decode hot path of SatPaingOo/joule, native to MI355X.

Router (softmax top-k, lowest-index ties) -> dispatch (counting sort into
per-expert segments) -> fused Q4 grouped expert product (gate/up SwiGLU,
then down) -> weighted combine, as HIP kernels for gfx950 behind a C ABI
(include/joule_amd.h), over an expert store resident in HBM in the
reference's on-disk Q4 layout.

Modules
  q4_store  the Q4 format (quantise / dequantise, store writer, index)
  moe       HbmExpertStore: the store in HBM and layer_ffn_batch
  backend   KernelBackend plugin API with HipBackend (q4_gemv / q4_gemm)
  synth     seeded synthetic workloads
  build     hipcc build of libjoule_amd.so
"""

__version__ = "0.1.0"
