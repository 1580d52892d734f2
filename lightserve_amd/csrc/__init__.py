"""HIP sources and the in-tree build script of liblsfa_gfx950.so."""
