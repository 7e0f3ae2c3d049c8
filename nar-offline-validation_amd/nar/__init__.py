"""Drop-in package for the reference's `nar` modules on the rotate-and-quantize path.

Provided here: `nar.kernels.r4_fused_v2` and `nar.kernels.r4_fused_v3` (the E17
launchers, backed by libnarhip.so) and `nar.fold_signed_permutation` (the
offline fold of the factors).  The package path is extended with any other
`nar` directory on sys.path, so that with this package first and the
reference checkout after it, the reference's remaining modules (experiment
drivers, hooks) import as before and pick these up.
"""

from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
