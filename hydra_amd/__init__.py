"""HydraHIP: the mixture-of-experts layer of Hydra, MI355X-native (gfx950).

Submodules:
  formats  layer descriptions, enums and expert blob layouts (no GPU needed)
  synth    the deterministic synthetic weight / input generator (no GPU needed)
  _lib     ctypes binding of libhydra_hip.so (the C ABI of include/hydra_hip.h)
  layer    MoELayer / Context: device-resident layer over the C ABI (needs torch + a GPU)
  build    hipcc build of libhydra_hip.so for gfx950
"""
__all__ = ["formats", "synth"]
