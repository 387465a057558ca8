"""CPU oracle of the COMP decode path: test infrastructure only (tests/, __graft_entry__.smoke(), bench.py's
cpu_baseline leg).  The product package comp_amd never imports it."""
