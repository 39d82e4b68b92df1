"""CPU oracle for the afhip parity tests (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker. The product (libafhip and the afhip
package) never loads it.
"""
