"""CPU oracle of the quantized MoE-FFN path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as the
reference its result is compared with) and bench.py's cpu_baseline leg.  Nothing under localmoe35ba3b_amd/
may import it.  See moe_oracle.py for the restated reference arithmetic and
tests/test_oracle_pins.py for the checks that pin each function.
"""
