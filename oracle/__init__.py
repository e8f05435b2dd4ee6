"""CPU oracle of the Wan DiT attention path (test infrastructure only; see oracle/ref.py)."""
