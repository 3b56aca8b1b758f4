"""CPU oracle for momij's verify step -- test infrastructure only (see oracle/oracle.py)."""
