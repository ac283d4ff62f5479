"""wisp (MI355X build): the fused group-wise expert dequant+GEMV path of WiSP Runtime
(imronpuji/wisp-runtime) on gfx950, behind the same module surface
(wisp.quant, wisp.kernels, wisp.cache_core, wisp.cache, wisp.store)."""

__version__ = "0.1.0"
