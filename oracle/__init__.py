"""CPU oracle of the PoPE attention path -- test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
never by the product package.  See pope_oracle.py for what each function
restates and how it is pinned.
"""
