"""CPU oracle for the dense-contraction path: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the checker. The product (torchvulkan_amd) never
imports, links or runs anything under oracle/.
"""
