"""The FP32 Gumbel noise of the certified draws, checked over all 2^32 Philox words.

The draws prune and certify with three facts about gumbel32 / gumbel_upper
(exactsample/csrc/es_device.h) that depend on the device's logf, log1pf
and __logf: |gumbel32(w) - G(w)| <= 2^-19 (1 + |G|), gumbel_upper(w) >= G(w),
and G(w) < 22.875, with G = -log(-log u), u = (w + 0.5) / 2^32, in FP64. The
library's es_check_gumbel makes the three checks on the device (the role of
the reference's tests/exhaustive/gumbel_bound.cu); the noise range it reports
is compared with its closed form at the two extreme words.
"""
import ctypes
import math
import struct

import numpy as np
import pytest

from exactsample import capi


def from_key(k):
    bits = k & ((1 << 63) - 1) if k >> 63 else (~k) & ((1 << 64) - 1)
    return struct.unpack("<d", struct.pack("<Q", bits))[0]


def noise(w):
    """G(w) in FP64 with the tail through log1p (the device self-test's form)."""
    e = -math.log((w + 0.5) / 2**32) if w < 2**31 else -math.log1p(-((2**32 - 1 - w) + 0.5) / 2**32)
    return -math.log(e)


def test_noise_range_closed_form():
    # The extreme words give the extreme noise: G is increasing in u.
    assert noise(0) == pytest.approx(-math.log(math.log(2**33)), rel=1e-15)
    assert -3.1300 < noise(0) < -3.1299
    assert 22.8738 < noise(2**32 - 1) < 22.8739 < 22.875
    words = np.sort(np.random.default_rng(1).integers(0, 2**32, size=2000))
    values = [noise(int(w)) for w in words]
    assert all(a <= b for a, b in zip(values, values[1:]))


def test_rejects_bad_ranges_without_a_launch():
    lib = capi.load()
    fake = ctypes.c_void_p(1 << 20)
    assert lib.es_check_gumbel(0, 1, None, None) == 1
    assert lib.es_check_gumbel(2**32 + 1, 0, fake, None) == 2
    assert lib.es_check_gumbel(5, 2**32, fake, None) == 2
    assert lib.es_check_gumbel(0, 1, ctypes.c_void_p((1 << 20) + 4), None) == 5


@pytest.mark.gpu
def test_all_words_on_the_device(hip_device):
    import torch

    lib = capi.load()
    report = torch.empty(8, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    chunk = 1 << 30
    totals = np.zeros(4, dtype=np.uint64)
    worst, slack, hi, lo = 0.0, math.inf, -math.inf, math.inf
    for first in range(0, 1 << 32, chunk):
        code = lib.es_check_gumbel(first, chunk, ctypes.c_void_p(report.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
        assert code == 0, (lib.es_error_string(code), lib.es_last_hip_error())
        words = [int(x) & ((1 << 64) - 1) for x in report.cpu().tolist()]
        totals += np.array(words[:4], dtype=np.uint64)
        worst = max(worst, struct.unpack("<d", struct.pack("<Q", words[4]))[0])
        slack, hi, lo = min(slack, from_key(words[5])), max(hi, from_key(words[6])), min(lo, from_key(words[7]))
        print(f"words [{first}, {first + chunk}): error/bound <= {worst:.4f}, screen margin >= {slack:.3g}", flush=True)
    checked, bad_error, bad_screen, bad_range = (int(x) for x in totals)
    assert checked == 1 << 32
    assert (bad_error, bad_screen, bad_range) == (0, 0, 0)
    assert worst <= 1.0 and slack >= 0.0
    assert hi == pytest.approx(noise(2**32 - 1), rel=1e-14) and lo == pytest.approx(noise(0), rel=1e-14)


def test_weight_check_rejects_bad_ranges_without_a_launch():
    lib = capi.load()
    fake = ctypes.c_void_p(1 << 20)
    assert lib.es_check_weights(0, 1, None, None) == 1
    assert lib.es_check_weights(2**32 + 1, 0, fake, None) == 2
    assert lib.es_check_weights(0, 1, ctypes.c_void_p((1 << 20) + 4), None) == 5


@pytest.mark.gpu
def test_fp32_weights_and_their_bound_on_the_device(hip_device):
    """Every FP32 x in [-40, 0]: |expf(x) / exp(x) - 1| <= 2.9e-7; and 2^31
    pseudo-random (v, M, T): the x32 formation within 1.8e-7 |x| and the
    certified sums' bound |expf(x32) / exp(x) - 1| <= X_ERR (1 + |x|), X_ERR =
    4.8e-7 (the constant the kernels certify FP32 kept masses and min-p
    decisions with)."""
    import torch

    lib = capi.load()
    report = torch.empty(8, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream()
    chunk, total = 1 << 29, 1 << 31
    sums = np.zeros(5, dtype=np.uint64)
    worst = [0.0, 0.0, 0.0]
    for first in range(0, total, chunk):
        code = lib.es_check_weights(first, chunk, ctypes.c_void_p(report.data_ptr()),
                                    ctypes.c_void_p(stream.cuda_stream))
        assert code == 0, (lib.es_error_string(code), lib.es_last_hip_error())
        words = [int(x) & ((1 << 64) - 1) for x in report.cpu().tolist()]
        sums += np.array(words[:4] + [words[7]], dtype=np.uint64)
        for j in range(3):
            worst[j] = max(worst[j], struct.unpack("<d", struct.pack("<Q", words[4 + j]))[0])
        print(f"indices [{first}, {first + chunk}): expf error <= {worst[0]:.3g}, formation <= {worst[1]:.3g} |x|, "
              f"combined <= {worst[2]:.4f} of the bound", flush=True)
    checked, bad_exp, bad_form, bad_comb, n_exp = (int(x) for x in sums)
    assert checked == total
    assert n_exp == 0x42200001  # every FP32 x from -0 to -40
    assert (bad_exp, bad_form, bad_comb) == (0, 0, 0)
    assert worst[0] <= 2.9e-7 and worst[1] <= 1.8e-7 and worst[2] <= 1.0
