"""gfx950 backend: ctypes binding of libtrnsparse_hip.so and the op dispatch."""
