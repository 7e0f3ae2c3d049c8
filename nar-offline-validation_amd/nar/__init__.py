"""Drop-in package for the reference's `nar` kernel modules on MI355X.

Only the rotate-and-quantize path is provided: `nar.kernels.r4_fused_v2` and
`nar.kernels.r4_fused_v3` (the E17 launchers), backed by libnarhip.so.
"""
