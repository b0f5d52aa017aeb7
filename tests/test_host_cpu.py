"""Host logic of the training package on the CPU: curriculum, configs, collator, layout helpers,
LoRA target resolution, resume validation and objective combination (reference error types)."""
import json

import pytest
import torch

from oracle import hashing as H
from oracle import layout as olay
from uno_amd import model as umodel
from uno_amd.training import config as ucfg
from uno_amd.training import curriculum as ucur
from uno_amd.training import data as udata
from uno_amd.training import losses as ulosses
from uno_amd.training import modeling as umod
from uno_amd.training import lora as ulora
from uno_amd.training import trainer as utrain

# The released recipe: 524,288 tokens/step; stage budgets in tokens (block size -> tokens).
RELEASED = {"tokens_per_step": 524288, "sequence_length": 4096, "global_batch_size": 128,
            "total_tokens": 14745600000, "seed": 20260813,
            "stages": [{"block_size": 2, "tokens": 2457862144}, {"block_size": 4, "tokens": 2457337856},
                       {"block_size": 6, "tokens": 2457862144}, {"block_size": 8, "tokens": 2457337856},
                       {"block_size": 12, "tokens": 2457862144}, {"block_size": 16, "tokens": 2457337856}]}


def test_curriculum_released_schedule():
    plan = ucur.BlockCurriculumPlan.from_dict(RELEASED)
    assert plan.max_steps == 28125
    assert [s.end_step for s in plan.stages] == [4688, 9375, 14063, 18750, 23438, 28125]
    assert plan.stage_for_step(0).block_size == 2
    assert plan.stage_for_step(4687).block_size == 2
    assert plan.stage_for_step(4688).block_size == 4
    assert plan.stage_for_step(28124).block_size == 16
    with pytest.raises(ValueError):
        plan.stage_for_step(28125)
    assert plan.checkpoint_reasons[14063] == "completed_block_size_6"
    assert len(plan.sha256()) == 64


@pytest.mark.parametrize("mutate", [
    lambda r: r.update(tokens_per_step=1000),
    lambda r: r.update(stages=[]),
    lambda r: r["stages"].reverse(),
    lambda r: r.update(total_tokens=5),
    lambda r: r.update(replay={"x": 1}),
    lambda r: r.update(seed="x"),
])
def test_curriculum_rejects_bad_plans(mutate):
    raw = json.loads(json.dumps(RELEASED))
    mutate(raw)
    with pytest.raises(ValueError):
        ucur.BlockCurriculumPlan.from_dict(raw)


def test_curriculum_hash_matches_reference_vectors(tmp_path):
    """sha256() of the released schedule and of synthetic schedules equals the reference's own
    (tests/golden/curriculum_vectors.json, written by tests/golden/make_curriculum_vectors.py from the
    reference's training/curriculum.py): boundary checkpoints of either implementation validate in the
    other. Also the stage boundaries and the manifest, key for key; from_yaml and from_dict agree."""
    from pathlib import Path

    import yaml
    vec = json.loads((Path(__file__).parent / "golden" / "curriculum_vectors.json").read_text())
    cases = [vec["released"], *vec["synthetic"]]
    assert len({c["sha256"] for c in cases}) == len(cases)
    for i, case in enumerate(cases):
        plan = ucur.BlockCurriculumPlan.from_dict(case["input"])
        assert [s.end_step for s in plan.stages] == case["end_steps"]
        assert plan.max_steps == case["max_steps"]
        assert plan.manifest() == case["manifest"]
        assert plan.sha256() == case["sha256"]
        path = tmp_path / f"plan{i}.yaml"
        path.write_text(yaml.safe_dump(case["input"]))
        assert ucur.BlockCurriculumPlan.from_yaml(path).sha256() == case["sha256"]
    assert ucur.BlockCurriculumPlan.from_dict(RELEASED).sha256() == vec["released"]["sha256"]


def test_curriculum_yaml_missing_file(tmp_path):
    with pytest.raises(FileNotFoundError):
        ucur.BlockCurriculumPlan.from_yaml(tmp_path / "nope.yaml")


def test_objective_and_lora_settings_validation():
    ucfg.UnoObjectiveConfig().validate()
    assert ucfg.UnoObjectiveConfig().internal_ce_target == "clean_argmax"
    assert ucfg.UnoObjectiveConfig(ce_target="ground_truth").internal_ce_target == "data"
    for bad in (dict(ce_target="x"), dict(noise="mask"), dict(reverse_kl=False), dict(teacher_base_only=False),
                dict(ce_weight=-1.0), dict(tv_weight=0.0), dict(kl_weight=float("nan"))):
        with pytest.raises(ValueError):
            ucfg.UnoObjectiveConfig(**bad).validate()
    assert ucfg.LoraSettings("all", 64, None, 0.0).resolved_alpha == 1024
    for bad in (dict(rank=0), dict(alpha=0), dict(dropout=1.0)):
        kw = dict(target="all", rank=8, alpha=16, dropout=0.0)
        kw.update(bad)
        with pytest.raises(ValueError):
            ucfg.LoraSettings(**kw).validate()


def test_combine_objective_losses():
    obj = ucfg.UnoObjectiveConfig(ce_weight=0.5, kl_weight=0.25, tv_weight=2.0)
    out = utrain.combine_objective_losses(torch.tensor(2.0), torch.tensor(4.0), torch.tensor(1.0), obj)
    assert out.item() == pytest.approx(0.5 * 2 + 0.25 * 4 + 2.0)


def test_lora_targets():
    assert ulora.resolve_lora_targets("all") == ucfg.__dict__.get("SUPPORTED_LORA_MODULES",
                                                                  ulora.SUPPORTED_LORA_MODULES)
    assert ulora.resolve_lora_targets("qkvo") == ("q_proj", "k_proj", "v_proj", "o_proj")
    assert ulora.resolve_lora_targets("q_proj, down_proj") == ("q_proj", "down_proj")
    for bad in ("qq", "", "lm_head", "q_proj,q_proj"):
        with pytest.raises(ValueError):
            ulora.resolve_lora_targets(bad)


class _Tok:
    padding_side = "right"
    pad_token_id = 0


def test_collator_right_pads():
    col = udata.UnoDataCollator(_Tok(), sequence_length=6)
    out = col([{"input_ids": [5, 6, 7], "labels": [-100, 6, 7]}, {"input_ids": [1] * 6, "labels": [1] * 6}])
    assert out["input_ids"][0].tolist() == [5, 6, 7, 0, 0, 0]
    assert out["labels"][0].tolist() == [-100, 6, 7, -100, -100, -100]
    assert out["attention_mask"][0].tolist() == [1, 1, 1, 0, 0, 0]
    with pytest.raises(ValueError):
        col([])
    with pytest.raises(ValueError):
        col([{"input_ids": [1] * 7, "labels": [1] * 7}])
    with pytest.raises(ValueError):
        col([{"input_ids": [1, 2], "labels": [1]}])

    class Left(_Tok):
        padding_side = "left"
    with pytest.raises(ValueError):
        udata.UnoDataCollator(Left())


def test_layout_helpers_match_oracle():
    pos = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 7], [0, 1, 2, 0, 1, 0, 1, 2]])
    ours = umodel.calculate_token_nums(pos)
    ref = olay.calculate_token_nums(pos)
    assert [t.tolist() for t in ours] == [t.tolist() for t in ref]
    labels = torch.randint(0, 50, (2, 8))
    assert torch.equal(ulosses.shift_labels_for_next_token(labels, pos),
                       olay.shift_labels_for_next_token(labels, pos))


def test_noise_key_matches_oracle():
    for seed, step in ((20260813, 0), (1, 7), (2 ** 63 + 5, 1000)):
        assert umodel.noise_key(seed, step) == int(H.step_key(seed, step))


def test_validate_uno_model_errors():
    class NotUno:
        config = type("C", (), {"block_size": 4})()
    with pytest.raises(RuntimeError):
        umod.validate_uno_model(NotUno())
    with pytest.raises(RuntimeError):
        umod.configure_uniform_noise_config(type("C", (), {"noise": "mask"})())


def test_resume_validation(tmp_path):
    plan = ucur.BlockCurriculumPlan.from_dict(RELEASED)
    with pytest.raises(FileNotFoundError):
        utrain.validate_curriculum_resume(tmp_path, plan)
    (tmp_path / "uno_curriculum_state.json").write_text(json.dumps({"curriculum_sha256": "bad", "global_step": 4688}))
    with pytest.raises(ValueError):
        utrain.validate_curriculum_resume(tmp_path, plan)
    (tmp_path / "uno_curriculum_state.json").write_text(
        json.dumps({"curriculum_sha256": plan.sha256(), "global_step": 100}))
    with pytest.raises(ValueError):
        utrain.validate_curriculum_resume(tmp_path, plan)
    (tmp_path / "uno_curriculum_state.json").write_text(
        json.dumps({"curriculum_sha256": plan.sha256(), "global_step": 4688}))
    utrain.validate_curriculum_resume(tmp_path, plan)


def test_portable_adapter_metadata(tmp_path):
    (tmp_path / "adapter_config.json").write_text(json.dumps({"base_model_name_or_path": "/cache/x"}))
    (tmp_path / "README.md").write_text("---\nbase_model: /cache/x\n---\n")
    ulora.make_saved_adapter_portable(tmp_path)
    cfg = json.loads((tmp_path / "adapter_config.json").read_text())
    assert cfg["base_model_name_or_path"] == "s-sahoo/uno-qwen3-8B"
    assert "base_model: s-sahoo/uno-qwen3-8B" in (tmp_path / "README.md").read_text()


def test_packing_collator_layout():
    """First-fit packing: every example lands once, in order, in one row; positions restart at each
    example; the unused tail is its own all-padding segment with IGNORE_INDEX labels."""
    class Tok:
        pad_token_id = 0
    lengths = [5, 3, 7, 2]
    feats = [{"input_ids": list(range(100 * (i + 1), 100 * (i + 1) + n)),
              "labels": [-100] + list(range(100 * (i + 1) + 1, 100 * (i + 1) + n))} for i, n in enumerate(lengths)]
    col = udata.UnoPackingCollator(Tok(), sequence_length=8)
    assert col.plan(lengths) == [[0, 1], [2], [3]]
    out = col(feats)
    assert out["input_ids"][0].tolist() == feats[0]["input_ids"] + feats[1]["input_ids"]
    assert out["position_ids"][0].tolist() == [0, 1, 2, 3, 4, 0, 1, 2]
    assert out["position_ids"][1].tolist() == [0, 1, 2, 3, 4, 5, 6, 0]
    assert out["position_ids"][2].tolist() == [0, 1, 0, 1, 2, 3, 4, 5]
    assert out["labels"][2].tolist() == feats[3]["labels"] + [-100] * 6
    assert out["attention_mask"][1].tolist() == [1] * 7 + [0]
    segs = [t.tolist() for t in olay.calculate_token_nums(out["position_ids"])]
    assert segs == [[5, 3], [7, 1], [2, 6]]
    # fixed row count: padded with all-padding rows, an error when too small
    assert udata.UnoPackingCollator(Tok(), sequence_length=8, rows=4)(feats)["input_ids"].shape == (4, 8)
    with pytest.raises(ValueError):
        udata.UnoPackingCollator(Tok(), sequence_length=8, rows=2)(feats)
    with pytest.raises(ValueError):
        col([{"input_ids": [1] * 9, "labels": [1] * 9}])
