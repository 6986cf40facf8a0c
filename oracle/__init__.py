"""CPU oracle of the quantized-matmul path.  Test infrastructure only (see holo_oracle.c)."""
