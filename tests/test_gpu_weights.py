"""Models loaded from weights files (ien_model_load, weight_file.rs format)
on the GPU: a file written from a model's tensors runs bit for bit like
the same tensors passed in memory (ien_model_from_tensors), in f32 and with
the export tools' --half matrices (against the f16-rounded tensors); a
file with a missing, misshapen or unused tensor is refused with the
reference's message (weight_file.rs:119-146)."""

import numpy as np
import pytest

import synthetic
import weights as W

pytestmark = pytest.mark.gpu


def inputs(kind):
    import ien

    if kind == ien.MODEL_REALESRGAN:
        return synthetic.esrgan_image(24, 32, seed=1), None
    if kind == ien.MODEL_SCUNET:
        return synthetic.scunet_image(64, 64, seed=2), None
    if kind == ien.MODEL_LAMA:
        return synthetic.lama_image(32, 40, seed=3), synthetic.lama_mask(32, 40, seed=4)
    return synthetic.birefnet_image(64, seed=5), None


def cases():
    import ien

    return [(ien.MODEL_REALESRGAN, W.MAGIC_REALESRGAN, synthetic.esrgan_tensors),
            (ien.MODEL_SCUNET, W.MAGIC_SCUNET, lambda: synthetic.scunet_tensors(init="fan")),
            (ien.MODEL_LAMA, W.MAGIC_LAMA, synthetic.lama_tensors),
            (ien.MODEL_BIREFNET, W.MAGIC_BIREFNET, lambda: synthetic.birefnet_tensors(init="fan"))]


@pytest.mark.parametrize("which", range(4))
@pytest.mark.parametrize("half", [False, True])
def test_file_equals_tensors(ctx, tmp_path, which, half):
    import ien

    kind, magic, make = cases()[which]
    tensors = make()
    rule = W.matrices_half if half else (lambda n, a: False)
    path = tmp_path / "model.weights"
    W.write(path, magic, tensors, rule)
    stored = {k: (v.astype(np.float16).astype(np.float32) if rule(k, v) else v) for k, v in tensors.items()}
    image, mask = inputs(kind)
    a = ien.Model(ctx, kind, path=path)
    got = a.run(image, mask=mask)
    a.free()
    b = ien.Model(ctx, kind, tensors=stored)
    want = b.run(image, mask=mask)
    b.free()
    assert np.isfinite(got).all() and np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_file_tensor_errors(ctx, tmp_path):
    import ien

    tensors = synthetic.esrgan_tensors()
    for change, message in (
            (lambda t: t.pop("body.66.bias"), "weights: body.66.bias: missing"),
            (lambda t: t.__setitem__("body.0.weight", t["body.0.weight"][:-1]),
             "weights: body.0.weight: shape [26,64,], expected [27,64,]"),
            (lambda t: t.__setitem__("extra", np.zeros(3, np.float32)), "weights: extra: not used by this model")):
        t = dict(tensors)
        change(t)
        path = tmp_path / "bad.weights"
        W.write(path, W.MAGIC_REALESRGAN, t)
        with pytest.raises(ien.IenError) as e:
            ien.Model(ctx, ien.MODEL_REALESRGAN, path=path)
        assert e.value.status == ien.ERR_WEIGHTS and str(e.value) == message, str(e.value)
    path = tmp_path / "scunet.weights"
    W.write(path, W.MAGIC_SCUNET, tensors)
    with pytest.raises(ien.IenError) as e:
        ien.Model(ctx, ien.MODEL_REALESRGAN, path=path)
    assert str(e.value) == "weights: not a REALESRG weights file"
