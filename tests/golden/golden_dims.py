"""Dimensions of the reduced-width model fixture (model_small.npz)."""
SMALL = dict(n_nodes=16, feat=12, gcn=(8, 12, 16), dfc=(24, 8), prot=8, fus=(16, 8, 1), lut_nmax=138)
