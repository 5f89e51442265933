"""Python side of the MI355X speaker-embedding library: GGUF I/O, the seeded
synthetic inputs/models, and the ctypes binding of lib/libvoicedetect.so."""
