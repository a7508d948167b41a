"""MI355X-native (gfx950) decode-step hot path of an LLM serving runtime.

``runtime_amd.phase2`` mirrors the reference's ``runtime.phase2`` modules that sit
on the decode path, backed by the HIP kernels of ``libmxdecode.so``.
"""
