"""CPU oracle for the delta-rule core -- test infrastructure only (see gdn_oracle.py)."""
