"""Host logic of the lane order: which ray shapes are traced as images
(native.screen_layout) and when the training entries sort a flat batch."""
import torch

from vorotracing_amd import _C, native


def test_screen_layout():
    L = native.screen_layout
    assert L((600, 800)) == (1, 600, 800)
    assert L((3, 600, 800)) == (3, 600, 800)
    assert L((2, 3, 64, 48)) == (6, 64, 48)
    assert L((8, 8)) == (1, 8, 8)
    # the reference's full antialiasing: five rays per pixel, side by side in a row
    assert L((600, 800, 5)) == (1, 600, 4000)
    assert L((2, 600, 800, 5)) == (2, 600, 4000)
    # flat batches
    assert L((1000000,)) is None
    assert L((1000000, 5)) is None  # a training batch with five rays per pixel
    assert L((7, 800)) is None and L((800, 7)) is None
    assert L(()) is None


def test_image_dims_of_training_entries():
    r = lambda *s: torch.zeros(*s, 6)  # noqa: E731
    assert _C._image_dims(r(48, 64)) == (48, 64)
    assert _C._image_dims(r(48, 64, 5)) == (48, 320)
    assert _C._image_dims(r(4096, 5)) == (0, 0)
    assert _C._image_dims(r(4096)) == (0, 0)
    # CPU tensors never get a computed order (the entries then raise with the reference's messages)
    assert _C.default_ray_perm(r(1 << 17), torch.zeros(1 << 17, dtype=torch.uint32), 10) is None
