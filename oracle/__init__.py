"""CPU oracle of the LCSA path — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).
The product path (mlx-flashvsr-swift_amd/) never imports it."""
