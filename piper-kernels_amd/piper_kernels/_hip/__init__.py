"""Host-side plumbing for the gfx950 HIP library: target detection, build and ctypes loader."""
