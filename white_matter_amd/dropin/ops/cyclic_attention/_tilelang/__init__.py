"""The accelerated cyclic backend (backend="tilelang"), here the gfx950 HIP kernels."""
