"""Parity oracle: a CPU restatement of mashbox's quantized-linear exact path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, as the checker. The product
package mashbox_amd never imports it. Function-by-function citations and how each function is pinned are in
oracle/ref.py's header.
"""
