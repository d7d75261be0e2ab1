"""TaoMemory CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package: it is the checker (and the timed CPU baseline), never
part of the product path.
"""
