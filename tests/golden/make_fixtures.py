"""Write the golden fixtures under tests/golden/ from the reference's own data and test constants.

Run in the build container (it reads /root/reference, which does not exist on the GPU box):
    python tests/golden/make_fixtures.py
Nothing from the reference is imported or executed: demo.json is a data file,
and the known answers are constants transcribed from the reference's tests.
"""

import json
from pathlib import Path

HERE = Path(__file__).resolve().parent
REF = Path("/root/reference")


def main():
    demo = json.loads((REF / "website/data/demo.json").read_text())
    phases = [dict(offset=p["offset"], labels=p["labels"], edges=p["edges"]) for p in demo["phases"]]
    (HERE / "demo_t4k1_grid64.json").write_text(
        json.dumps(
            dict(
                source="reference website/data/demo.json (written by website/tools/generate_demo.py:17-35)",
                meaning="composite Hilbert grid 64, 4 tiles, K1 reciprocal bridges; labels per original "
                "64-token block; edges = sorted undirected (u, v) original-block bridge pairs per phase",
                phases=phases,
            )
        )
    )
    known = dict(
        build_plan_bridge_budget=dict(
            source="reference tests/test_plan.py:54-59 (build_plan defaults: grid 64, text 512, shared, K1)",
            tiles4=[24, 34, 32, 34],
            tiles16=[56, 57, 58, 55],
            physical_original_blocks_head=[15, 16, 47, 48],
        ),
        paired_hand_vector=dict(
            source="reference tests/test_paired_metadata.py:46-55",
            kv_indices=[[0, 1, 2, 4], [0, 1, 3, 5], [0, 1, 4, 5], [0, 1, 4, 5]],
            kv_counts=[4, 4, 4, 4],
            tokens=384,
            global_tokens=128,
            key_block_size=128,
            expect_indices_row0_head3=[0, 1, 2],
            expect_flags_row0_head3=[15, 9, 9],
        ),
        hilbert_grid2=dict(source="geometry.py:12-24 evaluated by hand for grid 2", order=[2, 0, 1, 3]),
    )
    (HERE / "known_answers.json").write_text(json.dumps(known, indent=1))


if __name__ == "__main__":
    main()
