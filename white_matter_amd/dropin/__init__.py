"""A drop-in ``white_matter/ops`` package tree (ops/) whose modules re-export
this package's operators under the reference's module paths
(src/white_matter/ops/**). Replacing the reference's ops/ directory by this
one leaves no module that registers the ``white_matter::`` operator names
with other kernels, so the HIP kernels run whatever the import order."""
