"""``omo_python_api``: drop-in for the reference's Python wrappers
(code/kernel/api/mxfp4.py, code/kernel/api/mxfp4_dequant.py), imported by the
TE integration as ``omo_python_api.mxfp4`` / ``omo_python_api.mxfp4_dequant``
(e.g. code/transformer_engine-2.8.diff:669)."""
