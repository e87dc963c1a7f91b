"""The physical GL-SDM layer stack around the HIP memory operator.

Mirrors S/layers/{common,attention,router,global_layer,stack}.py and the
residual block of S/baselines/block.py (S/ = projects/gl-sdm/src/gl_sdm/):
same module and parameter names, same arithmetic and the same chunk clock.
Dense projections, normalisation and the local windowed attention are
PyTorch (hipBLASLt GEMMs, SDPA); every memory step (route, snapshot read,
proposal, commit) runs in libglsdm.so.
"""
