"""CPU oracle of the int4-dequant GEMM (test infrastructure only; see q4_oracle.h)."""
