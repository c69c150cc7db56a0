"""CPU oracle (test infrastructure): restatements of the reference's SoA
decode and GEMV used only by tests/, smoke() and bench.py's CPU baseline."""
