"""Test infrastructure: the CPU oracle for the attention path (see attention.py).
Never imported by the library under hackable-lm_amd/."""
