"""CPU oracle of the decode-time linear layers: test infrastructure only.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may
import this package, and only as the checker.  The product path
(breeze-tts-2_amd/) never calls it.
"""
