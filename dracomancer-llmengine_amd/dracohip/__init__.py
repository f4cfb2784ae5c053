"""dracohip -- host-side Python layer of the MI355X decode path.

lib      ctypes binding of libdraco_hip.so (the HIP kernels behind the m5_/m6_ C ABI)
models   seeded synthetic GGUF-format models of the benchmark configurations
driver   the llama-family driver (descriptor building and token loop of
         src/smol_engine.py), usable against any library exporting the m6 ABI
"""
