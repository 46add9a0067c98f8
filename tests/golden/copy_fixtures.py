"""Copy the reference's golden data for the CTC decode, DB post-process,
resize, crop and recogniser-input stages into this directory.

Data only (inputs and expected outputs written by the reference's own
fixture generator from OpenCV, pyclipper, RapidOCR and numpy); run once
where the reference tree is mounted:

    python tests/golden/copy_fixtures.py /root/reference/tests/fixtures
"""
import json
import shutil
import sys
from pathlib import Path

KEYS = ["resize", "det_input", "contours", "boxes", "min_area_rect", "unclip", "crops",
        "rec_input", "ctc"]


def main(src: Path, dst: Path) -> None:
    fx = json.loads((src / "fixtures.json").read_text())
    keep = {k: fx[k] for k in KEYS}
    files = {"characters.txt", "noise.npy", "page.npy", keep["det_input"]["file"],
             keep["boxes"]["file"]}
    files |= {c["file"] for c in keep["resize"]}
    files |= {c["file"] for c in keep["contours"]}
    files |= {c["file"] for c in keep["crops"]}
    for c in keep["rec_input"]:
        files |= {c["crop"], c["input"]}
    for c in keep["ctc"]:
        files |= {c["stem"] + "_argmax.npy", c["stem"] + "_maxprob.npy"}
    for f in sorted(files):
        shutil.copyfile(src / f, dst / f)
    (dst / "fixtures.json").write_text(json.dumps(keep, ensure_ascii=False, separators=(",", ":")))
    print(f"{len(files) + 1} files into {dst}")


if __name__ == "__main__":
    main(Path(sys.argv[1]), Path(__file__).resolve().parent)
