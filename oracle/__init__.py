"""CPU oracle of the grouped-GEMM path; test infrastructure only (tests/, smoke(), bench cpu_baseline)."""
