"""vaayu_amd: Vaayu's packed-expert routed-MoE path, built for MI355X (gfx950).

Drop-in modules (same entry points as the reference's):
  vaayu_amd.packed_expert_kernels   decode / prefill kernels, verdicts, graph, installer
  vaayu_amd.moe_patch               packed-blob formats, dequant, fixed-order accumulate
  vaayu_amd.block_formats           FP8 block-scaled and MXFP4 expert blobs
The kernels are HIP for gfx950 behind the C ABI of include/vaayu_amd.h
(vaayu_amd/libvaayu_amd.so, built by `python -m vaayu_amd.build`).
"""
__version__ = "0.1.0"
