"""HIP (gfx950) kernels behind the reference's nar/kernels launcher API."""

from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
