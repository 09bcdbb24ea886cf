"""Host-side Python mirror of the MI355X matmul backend for sam3.c.

``abi`` restates sam3.c's boundary structs, ``synth`` the seeded input
generator shared with the CPU oracle, and ``hip`` binds libsam3hip.so.
"""
