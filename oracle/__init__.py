"""CPU oracle of the MoE expert path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker; the product package moeinfra_amd never does.
"""
