"""CPU oracle for the INT8 group-quant matmul path (test infrastructure only; see sq8_oracle.c)."""
