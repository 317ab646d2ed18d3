"""gfx950 HIP kernels behind the reference's paged-attention operator API."""
