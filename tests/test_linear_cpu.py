"""Host-side checks of SRLinear (muon_sr_amd/linear.py); no GPU."""
def test_wgrad_shape_fits_matches_the_kernel_preconditions():
    """SRLinear's fallback predicate covers every operand check of
    msr_linear_wgrad_sr_accum, so unfit shapes return dW to autograd instead of
    raising inside backward."""
    from muon_sr_amd.linear import wgrad_shape_fits as fits
    ok = dict(out_f=4096, in_f=4096, tokens=8192, ldx=4096, ldy=4096, x_ptr=1 << 20, dy_ptr=1 << 21)
    assert fits(**ok)
    assert not fits(**dict(ok, in_f=4096 + 8))          # features not multiples of 256
    assert not fits(**dict(ok, tokens=8192 + 64))       # tokens not a multiple of 128
    assert not fits(**dict(ok, x_ptr=(1 << 20) + 2))    # misaligned view
    assert not fits(**dict(ok, ldy=4096 + 4))           # row stride not a multiple of 8
    assert not fits(**dict(ok, ldx=2048))               # row stride shorter than the row
    # LM head 4096 -> 128256: dy spans 2 GiB from 8,372 tokens (rounded to 128s: 8,448)
    head = dict(ok, out_f=128256 // 256 * 256 + 256, ldy=128256 // 256 * 256 + 256)
    head_ok = dict(head, tokens=8192)
    assert fits(**head_ok)
    assert not fits(**dict(head, tokens=8448))
    # Llama-3-8B MLP (14336 features) at 74,899 tokens or more
    mlp = dict(ok, in_f=14336, ldx=14336)
    assert fits(**dict(mlp, tokens=74880))
    assert not fits(**dict(mlp, tokens=75008))
