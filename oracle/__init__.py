"""CPU oracle of the paged-KV path. Test infrastructure only (tests/, smoke(), bench.py's
cpu_baseline leg); never imported by the product package."""
