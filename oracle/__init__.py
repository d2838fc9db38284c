"""CPU fp32 oracle of the reference denoise loops (test infrastructure only)."""
