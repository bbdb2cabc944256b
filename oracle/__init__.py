"""CPU oracle: TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py cpu_baseline)."""
