"""TEST INFRASTRUCTURE ONLY: CPU oracle for the Q4_K/Q6_K path (see oracle/oracle.py)."""
