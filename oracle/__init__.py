"""CPU oracle of the MoE hot path -- test infrastructure only (the checker
for ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU
baseline); the product never imports it."""
