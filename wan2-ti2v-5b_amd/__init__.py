"""MI355X (gfx950) attention hot path of the Wan2.2-TI2V-5B DiT.

Layout of the package:
  csrc/          HIP kernels (flash attention, QK-RMSNorm / RoPE prep) and the C ABI
                 declared in include/wan_attn.h, built into libwan_attn.so by build.py
  _native.py     ctypes binding of that C ABI
  ops.py         torch.library custom ops over it (wan_hip::*)
  rope.py        3D-RoPE angle tables (host side, once per grid)
  attention.py   attention() dispatch of wan/modules/attention.py
  fast_dit.py    the FAST_ATTN_IMPL-selected backends, the block forward and the batched-CFG
                 DiT of models/fast_dit.py, and the denoising loop
  model.py       the WanModel parameter tree (random initialisation for synthetic runs)
  unipc.py       the flow-matching UniPC sampler that drives the denoising loop

The directory name is not a Python identifier; load it as the module
`wan2_ti2v_5b_amd` (see load_package() in __graft_entry__.py).
"""
from . import _native, ops, rope  # noqa: F401
from . import attention, fast_dit, model, unipc  # noqa: F401

__all__ = ["_native", "ops", "rope", "attention", "fast_dit", "model", "unipc"]
