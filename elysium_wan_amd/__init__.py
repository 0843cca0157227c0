"""elysium_wan_amd -- the per-stage mixed-precision update path of
elysium-wan (wantrain) as MI355X-native HIP kernels behind wantrain's own
Python signatures.

Modules mirror the reference's:
  optim   -- runtime/optim.py   (build, hparams, state_bytes_per_param, the
             fused clip + AdamW + bf16 working copy, clip_grad_norm_)
  fp8     -- model/fp8.py       (scale_exp, quantize, dequantize, roundtrip,
             recover_exp)
  pieces  -- runtime/pieces.py  (cast_piece, fold_start, fold_add, fold)
  accumulate -- runtime/accumulate.py (OrderedAccumulator: the ordered
             microbatch fold, with the last part optionally left for the
             fused update)
  planes  -- codec/planes.py    (encode, decode, encode_scaled_fp8: the
             byte-plane and scaled-fp8 wires)
  fp8_planes -- codec/fp8_planes.py (encode, decode: the e4m3 nibble wire)
  f32_planes -- codec/f32_planes.py (encode, decode: the fp32 gradient wire)
  boundary -- model/gpt.py:284-317 (narrow, Boundary: the codec's caller)
The kernels live in libelyhip.so (C ABI: include/ely.h), built by
elysium_wan_amd.build for gfx950.
"""

from . import accumulate, boundary, f32_planes, fp8, fp8_planes, optim, pieces, planes  # noqa: F401

__all__ = ["accumulate", "boundary", "f32_planes", "fp8", "fp8_planes", "optim", "pieces", "planes"]
