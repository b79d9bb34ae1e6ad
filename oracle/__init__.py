"""CPU oracle of the ConvRot contract -- test infrastructure only (see oracle.py)."""
