"""MI355X-native decoder-LM forward/backward step with the call surface of resihp.

``resihp.model``, ``resihp.reference``, ``resihp.parallel.tp`` and
``resihp.parallel.reshard`` keep the names, signatures and error behaviour of
ksqbxm/resihp-reproduction; their compute runs in the gfx950 HIP library
``libresihp_hip.so`` (C ABI: include/resihp_hip.h) via :mod:`resihp.ops`.
"""

__all__ = ["config", "model", "ops", "reference"]
