"""GPU parity of the output stage (src/decoder/output.rs) against the reference's PyTorch
vectors and the CPU oracle: align_corners resampling and the BT.709 picture -> RGB path, bit for
bit."""

import numpy as np
import pytest

import oracle
from tests.golden import zjtb
from zenjpegai_amd import _lib, model, nn, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    e = nn.Engine(0, "f32")
    yield e
    e.close()


@pytest.mark.parametrize("name,mode,cases", [("bicubic_align_corners", "bicubic", 6),
                                             ("bilinear_align_corners", "bilinear", 8)])
def test_resize_matches_reference_fixture_exactly(eng, name, mode, cases):
    t = zjtb.load(name)
    for i in range(cases):
        x, want = t[f"x{i}"], t[f"y{i}"]
        got = nn.resize(eng, x, want.shape[1], want.shape[2], mode)
        assert got.tobytes() == want.astype(np.float32).tobytes(), (i, x.shape, want.shape)


@pytest.mark.parametrize("mode", ["bicubic", "bilinear"])
@pytest.mark.parametrize("shape,out", [((2, 67, 45), (134, 90)), ((1, 135, 240), (270, 480)),
                                       ((3, 33, 47), (17, 24)), ((1, 1, 9), (1, 17)),
                                       ((2, 64, 1), (127, 3))])
def test_resize_matches_oracle(eng, mode, shape, out):
    x = np.random.default_rng(11).uniform(0, 255, shape).astype(np.float32)
    got = nn.resize(eng, x, *out, mode)
    fn = oracle.resize_bicubic if mode == "bicubic" else oracle.resize_bilinear
    assert np.array_equal(got, fn(x, *out))


def test_resize_rejects_empty_sizes(eng):
    with pytest.raises(_lib.HipError) as e:
        nn.resize(eng, np.zeros((1, 4, 4), np.float32), 0, 3)
    assert e.value.kind == "InvalidArgument"


def _rgb_picture(eng, h, w, sv, sh, seed):
    """A HOP Y+UV picture with float planes (bit_depth 0), two tiles."""
    lh, lw = -(-h // 16), -(-w // 16)
    py = synth.random_params("hop", "y", seed=seed, gain=0.5)
    puv = synth.random_params("hop", "uv", seed=seed, gain=0.5)
    tiles = model.synthesis_tiles(h, w, lh, lw, (128, 32))
    pic = model.Picture(eng, model.SynthesisPrimary.load(py, "hop", eng),
                        model.SynthesisSecondary.load(puv, "hop", eng), lh, lw, h, w, tiles, sv, sh)
    pic.upload(synth.latent(seed, "rgb/y", 160, lh, lw), synth.latent(seed, "rgb/uv", 96, lh, lw))
    pic.run()
    return pic


@pytest.mark.parametrize("h,w,sv,sh", [(136, 200, 2, 2), (128, 184, 1, 2), (96, 144, 1, 1)])
@pytest.mark.parametrize("bits", [8, 10])
def test_picture_rgb_matches_oracle(eng, h, w, sv, sh, bits):
    """4:2:0 and 4:2:2 chroma is bicubic-resampled to the luma size on the device, 4:4:4 goes
    straight through; RGB samples and float planes equal the oracle's on the same planes."""
    pic = _rgb_picture(eng, h, w, sv, sh, seed=41)
    y, u, v = pic.download()
    rgb, planes = pic.download_rgb(bits, planes=True)
    want_q, want_f = oracle.picture_rgb(y, u, v, bits)
    assert np.array_equal(planes, want_f)
    assert np.array_equal(rgb, want_q)
    assert rgb.max() <= (1 << bits) - 1
    # Without the float planes the samples are the same.
    assert np.array_equal(pic.download_rgb(bits), rgb)


def test_picture_rgb_needs_float_planes_and_8_or_10_bits(eng):
    pic = _rgb_picture(eng, 64, 64, 2, 2, seed=42)
    with pytest.raises(_lib.HipError) as e:
        pic.download_rgb(12)
    assert e.value.kind == "InvalidArgument"
    lh = lw = 4
    py = synth.random_params("hop", "y", seed=42, gain=0.5)
    puv = synth.random_params("hop", "uv", seed=42, gain=0.5)
    tiles = model.synthesis_tiles(64, 64, lh, lw, None)
    q = model.Picture(eng, model.SynthesisPrimary.load(py, "hop", eng),
                      model.SynthesisSecondary.load(puv, "hop", eng), lh, lw, 64, 64, tiles, 2, 2,
                      bit_depth=10)
    q.upload(synth.latent(42, "rgb/y", 160, lh, lw), synth.latent(42, "rgb/uv", 96, lh, lw))
    q.run()
    with pytest.raises(_lib.HipError) as e:
        q.download_rgb(10)
    assert e.value.kind == "InvalidArgument"
