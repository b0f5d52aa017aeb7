"""Pins the oracle's layout, label shift, hashing, noising and mask contract (CPU)."""
import numpy as np
import pytest
import torch

from oracle import bd, hashing as H, layout


def test_splitmix64_published_vector():
    # First outputs of the splitmix64 generator seeded with 0 (Vigna's reference generator).
    assert H.splitmix64_sequence(0, 5) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                                           0xF88BB8A8724C81EC, 0x1B39896A51A8749B]


def test_unit_float_and_noise_level_exact():
    assert H.unit_float(np.uint64(0)) == 0.0
    assert H.unit_float(np.uint64(0xFFFFFFFFFFFFFFFF)) == np.float32(1 - 2 ** -24)
    assert H.unit_float(np.uint64(1 << 63)) == 0.5
    assert H.noise_level(np.float32(0.0)) == np.float32(0.05)
    # largest u -> t stays below 1
    assert H.noise_level(np.float32(1 - 2 ** -24)) < 1.0
    # fp32 rounding: 0.5*0.95 -> 0.475 (rounded), + 0.05 (rounded)
    assert H.noise_level(np.float32(0.5)) == np.float32(np.float32(0.475) + np.float32(0.05))


def test_layout_single_and_packed_segments():
    ids = torch.zeros((2, 6), dtype=torch.long)
    pos = torch.tensor([[0, 1, 2, 3, 4, 5], [0, 1, 2, 0, 1, 0]])
    _, mp, region = layout.prepare_uno_layout(ids, pos)
    assert torch.equal(mp, pos)
    T, F = True, False
    assert region[0].tolist() == [T] * 6 + [F] * 6
    assert region[1].tolist() == [T, T, T, F, F, F, T, T, F, F, T, F]
    assert [x.tolist() for x in layout.calculate_token_nums(pos)] == [[6], [3, 2, 1]]
    _, _, r0 = layout.prepare_uno_layout(ids, None)
    assert torch.equal(r0, region[0:1].expand(2, -1))


def test_layout_rejects_bad_lengths():
    with pytest.raises(RuntimeError):
        layout.build_noisy_region_mask([torch.tensor([2, 2])], 5)


def test_shift_labels_hand_case():
    labels = torch.tensor([[-100, 5, 6, 7, 8, 9]])
    pos = torch.tensor([[0, 1, 2, 0, 1, 2]])
    out = layout.shift_labels_for_next_token(labels, pos)
    # boundary after index 2 (pos 2 >= 0) masks index 2; last column always masked
    assert out.tolist() == [[5, 6, -100, 8, 9, -100]]


def test_extract_regions_order():
    B, L, Hd = 1, 3, 2
    pos = torch.tensor([[0, 1, 0]])
    _, _, region = layout.prepare_uno_layout(torch.zeros(1, 3, dtype=torch.long), pos)
    hidden = torch.arange(2 * L * Hd, dtype=torch.float32).view(B, 2 * L, Hd)
    noisy, clean = layout.extract_uno_regions(hidden, region, L)
    # concat rows: [n0 n1 c0 c1 | n2 c2]
    assert noisy[0, :, 0].tolist() == [0, 2, 8]
    assert clean[0, :, 0].tolist() == [4, 6, 10]


@pytest.mark.parametrize("intra", ["bidirectional", "causal"])
@pytest.mark.parametrize("b", [1, 2, 3, 4, 6])
def test_dense_mask_matches_bruteforce(b, intra):
    pos = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 0, 1, 2, 3, 4], list(range(12))])
    assert torch.equal(bd.dense_mask(pos, b, intra), bd.dense_mask_bruteforce(pos, b, intra))


@pytest.mark.parametrize("L,b", [(64, 4), (60, 6), (40, 16)])
def test_causal_intra_block_pair_counts(L, b):
    """Causal in-block variant: a noisy query at in-block offset o sees o + 1 noisy keys, so a
    block of size n contributes n(n+1)/2 noisy-noisy pairs instead of n^2; the clean pairs are
    unchanged; with block size 1 both variants coincide."""
    pos = torch.arange(L)[None]
    _, noisy, _ = bd.concat_descriptors(pos)
    noisy = noisy[0]
    bi, ca = bd.dense_mask(pos, b)[0], bd.dense_mask(pos, b, "causal")[0]
    assert torch.equal(bi[~noisy], ca[~noisy])
    nn_bi = int(bi[noisy][:, noisy].sum())
    nn_ca = int(ca[noisy][:, noisy].sum())
    sizes = [min(b, L - s) for s in range(0, L, b)]
    assert nn_bi == sum(n * n for n in sizes)
    assert nn_ca == sum(n * (n + 1) // 2 for n in sizes)
    assert torch.equal(bd.dense_mask(pos, 1), bd.dense_mask(pos, 1, "causal"))


@pytest.mark.parametrize("L,b", [(64, 4), (96, 16), (60, 6), (48, 12), (40, 32)])
def test_dense_mask_pair_counts_closed_form(L, b):
    pos = torch.arange(L)[None]
    m = bd.dense_mask(pos, b)[0]
    _, noisy, _ = bd.concat_descriptors(pos)
    noisy = noisy[0]
    clean_pairs = int(m[~noisy].sum())
    noisy_pairs = int(m[noisy].sum())
    assert clean_pairs == L * (L + 1) // 2
    # noisy query in block k (start s_k, size b_k) sees s_k clean keys and b_k noisy keys
    expect = sum(min(b, L - s) * (s + min(b, L - s)) for s in range(0, L, b))
    assert noisy_pairs == expect
    # no clean query ever sees a noisy key
    assert not m[~noisy][:, noisy].any()


def _batch(B=2, L=64, prompt=16, V=4096, seed=0):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, V - 1, (B, L), generator=g)
    labels = ids.clone()
    labels[:, :prompt] = -100
    return ids, labels


def test_noising_invariants():
    ids, labels = _batch(B=4, L=512, prompt=64)
    pos = torch.arange(512)[None].expand(4, -1)
    prompt = labels == -100
    mask_id = 4095
    noised, nids, t = bd.noise_tokens(ids, pos, prompt, block_size=4, mask_token_id=mask_id, seed=7, step=3)
    assert not noised[prompt].any()
    assert ((t >= 0.05) & (t < 1.0)).all()
    tb = t.view(4, -1, 4)
    assert torch.equal(tb, tb[:, :, :1].expand_as(tb))          # one t per block
    rep = nids[noised]
    assert ((rep >= 1) & (rep < mask_id)).all()
    assert torch.equal(nids[~noised], ids[~noised])
    rate = noised[~prompt].float().mean().item()
    assert abs(rate - t[~prompt].mean().item()) < 0.03          # E[noised | t] = t
    again = bd.noise_tokens(ids, pos, prompt, block_size=4, mask_token_id=mask_id, seed=7, step=3)
    assert torch.equal(again[0], noised) and torch.equal(again[1], nids)
    other = bd.noise_tokens(ids, pos, prompt, block_size=4, mask_token_id=mask_id, seed=7, step=4)
    assert not torch.equal(other[0], noised)


def test_mask_noise_mode_and_concat():
    ids, labels = _batch(B=2, L=32, prompt=8)
    pos = torch.tensor([list(range(20)) + list(range(12)), list(range(32))])
    cids, cpos, mask, noised, t, p_mask = bd.prepare_for_bd_training(
        ids, pos, labels == -100, block_size=4, mask_token_id=4095, seed=1, step=0, noise="mask")
    _, _, region = layout.prepare_uno_layout(ids, pos)
    assert torch.equal(cids[~region].view(2, 32), ids)
    noisy_ids = cids[region].view(2, 32)
    assert (noisy_ids[noised] == 4095).all()
    assert torch.equal(cpos[region].view(2, 32), pos) and torch.equal(cpos[~region].view(2, 32), pos)
    assert p_mask.numel() == int(noised.sum())
    assert torch.equal(p_mask, t[noised])
    assert torch.equal(mask, bd.dense_mask(pos, 4))
