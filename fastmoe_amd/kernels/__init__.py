"""Import path of the reference (``fastmoe.kernels``)."""
