"""HIP (gfx950) kernels behind the reference's nar/kernels launcher API."""
