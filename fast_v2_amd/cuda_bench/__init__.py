"""Drop-in mirror of the reference's cuda_bench/ package (the fused sparse-path op)."""
