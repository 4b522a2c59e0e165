"""CPU oracle of the MoE block: test infrastructure only (tests/, smoke(), bench.py's
cpu_baseline leg). Never imported by the product package."""
