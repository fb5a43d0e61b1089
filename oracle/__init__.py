"""CPU oracle of the ragged-batch attention path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg import
this package. The product (sketchpad_amd/, include/) never does.
"""
