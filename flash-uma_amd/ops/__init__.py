"""Op layer of the FlashUMA hot path: torch.autograd.Functions with the reference's names
and signatures (ops/geom.py, ops/gather.py, ops/gating.py, ops/scatter.py, ops/ln_silu.py),
each calling the gfx950 kernels of libflashuma_hip.so through its C-ABI."""
