"""CPU oracle for MhcPre -- test infrastructure only (see oracle.py)."""
