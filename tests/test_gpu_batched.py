"""Multi-position MoE step (grouped int8 MFMA experts) through the C ABI, against the oracle's grouped integer order
bit for bit, and against the single-position GPU block for the routing."""
import numpy as np
import pytest

import moert
import oracle

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


SHAPES = [(1024, 512, 32, 8), (1536, 512, 40, 8), (1024, 128, 6, 2), (1536, 256, 64, 4)]


@pytest.mark.parametrize("hidden,inter,experts,k", SHAPES)
def test_batched_block_is_bit_identical_to_the_grouped_oracle(gpu, hidden, inter, experts, k):
    router = moert.synth_quantized(101, hidden, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(102, hidden, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(103, hidden, experts * hidden * inter, 0.02, moert.Q8_0)
    for zipf in (False, True):
        bias = moert.zipf_bias(experts, 7) if zipf else None
        blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, router_bias=bias)
        for m in (1, 3, 16, 17, 32):
            say(f"batched block hidden={hidden} inter={inter} E={experts} k={k} zipf={zipf} m={m}")
            x = moert.synth_normal(104, m, m * hidden).reshape(m, hidden)
            y, ids, w = blk.forward_batched(x)
            oy, oi, ow = oracle.moe_block_batched(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x,
                                                  bias=bias)
            assert ids.tolist() == oi.tolist(), m
            assert bits_equal(w, ow), m
            assert bits_equal(y, oy), m
            assert blk.experts_in_step() == len(np.unique(oi))
        blk.close()


def test_batched_block_with_every_position_on_the_same_experts(gpu):
    """All positions identical: every routed expert has m members (the widest member tile), and positions with
    zero input (all-zero activation blocks, scale 0)."""
    hidden, inter, experts, k = 1536, 512, 40, 8
    router = moert.synth_quantized(111, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(112, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(113, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0)
    for m, zero in ((16, False), (32, False), (5, True)):
        say(f"batched block identical positions m={m} zero={zero}")
        row = np.zeros(hidden, np.float32) if zero else moert.synth_normal(114, 0, hidden)
        x = np.tile(row, (m, 1))
        y, ids, w = blk.forward_batched(x)
        oy, oi, ow = oracle.moe_block_batched(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x)
        assert ids.tolist() == oi.tolist() and bits_equal(w, ow) and bits_equal(y, oy)
        assert blk.experts_in_step() == k
        assert (y == y[0]).all()
    blk.close()


def test_batched_routing_equals_the_single_position_gpu_block(gpu):
    hidden, inter, experts, k, m = 1536, 512, 40, 8, 16
    router = moert.synth_quantized(121, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(122, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(123, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    bias = moert.zipf_bias(experts, 9)
    blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, router_bias=bias)
    x = moert.synth_normal(124, 0, m * hidden).reshape(m, hidden)
    say("batched vs single-position routing")
    yb, ids, w = blk.forward_batched(x)
    for p in range(m):
        y1, i1, w1 = blk.forward(x[p])
        assert ids[p].tolist() == i1.tolist() and bits_equal(w[p], w1)
        # the two paths differ only by the 15-bit activation codes of the grouped path
        assert np.linalg.norm(yb[p] - y1) <= 2e-4 * np.linalg.norm(y1)
    blk.close()


def test_batched_block_refuses_bad_sizes(gpu):
    hidden, inter, experts, k = 1024, 128, 6, 2
    router = moert.synth_quantized(131, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(132, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(133, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0)
    with pytest.raises(moert.MoertError):
        blk.forward_batched(np.zeros((33, hidden), np.float32))
    blk.close()


@pytest.mark.parametrize("hidden,experts", [(1024, 32), (1536, 40)])
def test_batched_one_launch_is_bit_identical_to_the_grouped_oracle(gpu, hidden, experts):
    """moert_block_batched_kernel(1): the step as one launch over the XCDs, against the oracle and the four-kernel
    step of the same block, bit for bit (routing, weights, outputs, distinct experts), with and without a Zipf
    router bias, m = 1 .. 16."""
    inter, k = 512, 8
    router = moert.synth_quantized(121, hidden, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(122, hidden, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(123, hidden, experts * hidden * inter, 0.02, moert.Q8_0)
    for zipf in (False, True):
        bias = moert.zipf_bias(experts, 9) if zipf else None
        blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, router_bias=bias)
        for m in (1, 5, 16):
            say(f"one-launch block hidden={hidden} E={experts} zipf={zipf} m={m}")
            x = moert.synth_normal(124 + m, m, m * hidden).reshape(m, hidden)
            blk.batched_kernel(0)
            y0, i0, w0 = blk.forward_batched(x)
            blk.batched_kernel(1)
            y1, i1, w1 = blk.forward_batched(x)
            n1 = blk.experts_in_step()
            oy, oi, ow = oracle.moe_block_batched(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x,
                                                  bias=bias)
            assert i1.tolist() == oi.tolist() and bits_equal(w1, ow), m
            assert bits_equal(y1, oy), m
            assert bits_equal(y1, y0) and i1.tolist() == i0.tolist(), m
            assert n1 == len(np.unique(oi))
            # a second launch on the same buffers (the next epoch) gives the same bits
            y2, _, _ = blk.forward_batched(x)
            assert bits_equal(y2, y1), m
        blk.close()


def test_batched_one_launch_identical_positions_and_refusals(gpu):
    """One launch with every position on the same experts (m members each), zero inputs, and the shapes it refuses
    (more than 16 positions, ffn other than 512) with MOERT_E_CONFIG."""
    hidden, inter, experts, k = 1536, 512, 40, 8
    router = moert.synth_quantized(131, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(132, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(133, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0)
    blk.batched_kernel(1)
    for m, zero in ((16, False), (5, True)):
        say(f"one-launch identical positions m={m} zero={zero}")
        row = np.zeros(hidden, np.float32) if zero else moert.synth_normal(134, 0, hidden)
        x = np.tile(row, (m, 1))
        y, ids, w = blk.forward_batched(x)
        oy, oi, ow = oracle.moe_block_batched(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0, x)
        assert ids.tolist() == oi.tolist() and bits_equal(w, ow) and bits_equal(y, oy)
    with pytest.raises(moert.MoertError) as e:
        blk.forward_batched(np.zeros((17, hidden), np.float32))
    assert e.value.code == moert.E_CONFIG
    blk.close()
    small = moert.GpuBlock(1024, 256, 8, 2, moert.synth_quantized(135, 0, 8 * 1024, 0.02, moert.Q8_0),
                           moert.synth_quantized(136, 0, 8 * 2 * 256 * 1024, 0.02, moert.Q8_0),
                           moert.synth_quantized(137, 0, 8 * 1024 * 256, 0.02, moert.Q8_0), moert.Q8_0)
    with pytest.raises(moert.MoertError) as e:
        small.batched_kernel(1)
    assert e.value.code == moert.E_CONFIG
    small.close()


def test_batched_one_launch_failure_path_is_reported_and_cleared(gpu):
    """The one launch's bounded waits, each made to give up from the host (moert_block_fault_inject: the named wait
    looks for an epoch no launch writes): the step returns MOERT_E_DEVICE naming the wait, every workgroup ends
    (the next call runs), and with the mask cleared the next step equals the four kernels' bit for bit again. The
    hook is refused for the four-kernel mode and for unknown bits."""
    hidden, inter, experts, k, m = 1536, 512, 40, 8, 16
    router = moert.synth_quantized(141, 0, experts * hidden, 0.02, moert.Q8_0)
    gate_up = moert.synth_quantized(142, 0, experts * 2 * inter * hidden, 0.02, moert.Q8_0)
    down = moert.synth_quantized(143, 0, experts * hidden * inter, 0.02, moert.Q8_0)
    blk = moert.GpuBlock(hidden, inter, experts, k, router, gate_up, down, moert.Q8_0,
                         router_bias=moert.zipf_bias(experts, 144))
    x = moert.synth_normal(145, 0, m * hidden).reshape(m, hidden)
    y0, i0, w0 = blk.forward_batched(x)
    with pytest.raises(moert.MoertError) as e:
        blk.fault_inject(2)
    assert e.value.code == moert.E_CONFIG
    blk.batched_kernel(1)
    with pytest.raises(moert.MoertError) as e:
        blk.fault_inject(16)
    assert e.value.code == moert.E_CONFIG
    for bit, name in ((1, "router logits"), (2, "act vectors"), (4, "expert outputs"), (8, "input codes")):
        say(f"one-launch failure path: bit {bit} ({name})")
        blk.fault_inject(bit)
        with pytest.raises(moert.MoertError) as e:
            blk.forward_batched(x)
        assert e.value.code == moert.E_DEVICE and name in str(e.value), str(e.value)
        blk.fault_inject(0)
        y, ids, w = blk.forward_batched(x)
        assert ids.tolist() == i0.tolist() and bits_equal(w, w0) and bits_equal(y, y0), bit
    blk.close()
