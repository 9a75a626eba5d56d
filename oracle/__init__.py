"""CPU oracle of the FT path: test infrastructure only (tests, the smoke check
and the benchmark's CPU-baseline leg).  The product never imports it."""
