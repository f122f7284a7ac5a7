"""CPU oracle for the fused per-layer kernels: test infrastructure, never the product."""
