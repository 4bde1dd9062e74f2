"""The reference's evaluation protocol modules (``sparse_vggt.evaluation``,
e.g. ``pi3_reconstruction``) are not part of this build."""
raise ImportError("sparse_vggt.evaluation (the Pi3 reconstruction protocol) is not part of the vasc_amd build; "
                  "the Pi3 evaluator cannot compute its metrics with it")
