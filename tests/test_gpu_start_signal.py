"""The recurrence start signal used by the overlapped prefill schedule: the gated-delta
recurrence kernel raises it as it starts, the one-wave wait kernel returns on it or after
its time limit (forced here from the host with a flag that is never raised), and the
overlapped schedule gives the same bits as the same kernels run back to back (with a start
signal the recurrence is unsegmented, so against the sequential schedule's segmented
recurrence the memory output agrees to rounding)."""

import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu


def _elapsed_ms(fn):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def test_wait_returns_on_the_flag_or_after_the_limit(dev):
    from atma_amd.kernel import StartSignal
    sig = StartSignal(dev)
    sig.arm()
    sig.flag.fill_(sig.epoch)
    sig.wait(timeout_us=500_000)   # untimed: the first launch loads the library's code objects
    torch.cuda.synchronize()
    assert _elapsed_ms(lambda: sig.wait(timeout_us=500_000)) < 50.0   # already raised
    sig.arm()                                                        # never raised
    t = _elapsed_ms(lambda: sig.wait(timeout_us=3_000))
    assert 2.0 <= t < 500.0, t
    with pytest.raises(ValueError):
        torch.ops.atma_hip.wait_start_flag(sig.flag.float(), 1, 100)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_recurrence_raises_the_signal(dev, dtype):
    from atma_amd.kernel import StartSignal, chunk_gated_delta_rule
    g = torch.Generator(device=dev).manual_seed(0)
    B, T, H, d = 1, 200, 4, 64
    q, k, v = (torch.randn(B, T, H, d, device=dev, generator=g).to(dtype) for _ in range(3))
    gl = torch.randn(B, T, H, device=dev, generator=g)
    bl = torch.randn(B, T, H, device=dev, generator=g)
    sig = StartSignal(dev)
    ref = chunk_gated_delta_rule(q, k, v, gl, bl, scale=1.0, use_qk_l2norm_in_kernel=True,
                                 gate_bias=(3.9, 0.0), output_final_state=True)
    for _ in range(3):
        e = sig.arm()
        out = chunk_gated_delta_rule(q, k, v, gl, bl, scale=1.0, use_qk_l2norm_in_kernel=True,
                                     gate_bias=(3.9, 0.0), output_final_state=True, start_signal=sig)
        sig.wait()
        torch.cuda.synchronize()
        assert int(sig.flag.item()) == e
        assert torch.equal(out[0], ref[0]) and torch.equal(out[1], ref[1])
    e = sig.arm()   # no tokens: no recurrence launch, the wrapper raises the flag itself
    chunk_gated_delta_rule(q[:, :0], k[:, :0], v[:, :0], gl[:, :0], bl[:, :0], start_signal=sig)
    torch.cuda.synchronize()
    assert int(sig.flag.item()) == e


def test_overlap_policy(dev):
    from atma_amd.kernel import recurrence_pays_to_overlap as pays
    assert pays(1, 8, 128, torch.bfloat16, dev)        # 32 recurrence workgroups
    assert not pays(8, 8, 128, torch.bfloat16, dev)    # 256: one per CU
    assert pays(2, 8, 128, torch.bfloat16, dev)
    assert not pays(4, 8, 128, torch.float32, dev)     # fp32 slabs are 16 columns


@pytest.mark.parametrize("B,T", [(1, 4096), (2, 700)])
def test_overlapped_schedule_is_bitwise_the_sequential_one(dev, B, T):
    """The overlapped prefill (Polar waiting on the signal, memory on the side stream)
    against back to back, on bf16 inputs shaped like configs[2]'s heads."""
    from atma_amd.kernel import StartSignal, chunk_gated_delta_rule, polar_attention_fwd
    g = torch.Generator(device=dev).manual_seed(B * T)
    Hq, Hkv, d = 8, 2, 128
    q = torch.randn(B, Hq, T, d, device=dev, generator=g).bfloat16()
    k = torch.randn(B, Hkv, T, d, device=dev, generator=g).bfloat16()
    v = torch.randn(B, Hkv, T, d, device=dev, generator=g).bfloat16()
    zg = torch.randn(B, T, Hq, device=dev, generator=g)
    zb = torch.randn(B, T, Hq, device=dev, generator=g)
    n = torch.arange(1, T + 1, device=dev, dtype=torch.float32)
    p = dict(v_null=torch.randn(Hq, d, device=dev, generator=g) * 0.1,
             null_base=torch.full((Hq,), 2.0, device=dev), null_slope_raw=torch.full((Hq,), 0.5, device=dev),
             len_gain_raw=torch.full((Hq,), -1.0, device=dev), mag_beta_raw=torch.full((Hq,), -1.5, device=dev))

    def mem(sig=None):
        return chunk_gated_delta_rule(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), zg, zb,
                                      scale=1.0, use_qk_l2norm_in_kernel=True, gate_bias=(3.9, 0.0),
                                      output_final_state=True, start_signal=sig)

    sig, side = StartSignal(dev), torch.cuda.Stream(device=dev)
    main = torch.cuda.current_stream()
    c0, m0 = polar_attention_fwd(q, k, v, n, **p)
    sig.arm()
    o0, s0 = mem(sig)       # the overlapped schedule's plan, back to back (nobody waits)
    o2, s2 = mem()          # the sequential schedule's (segmented when T is long)
    assert rel_err(o2.float(), o0.float()) <= 1e-2 and rel_err(s2, s0) <= 1e-3
    for _ in range(3):
        sig.arm()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            o1, s1 = mem(sig)
        sig.wait()
        c1, m1 = polar_attention_fwd(q, k, v, n, **p)
        main.wait_stream(side)
        torch.cuda.synchronize()
        assert torch.equal(c0, c1) and torch.equal(m0, m1) and torch.equal(o0, o1) and torch.equal(s0, s1)
