"""CPU oracle of relmo's message-passing ops: test infrastructure only.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package, always as the checker / baseline, never as the path that
is measured or shipped.
"""
