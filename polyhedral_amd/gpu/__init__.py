"""Drop-in modules with the names of the reference's gpu/ directory.

Drivers written against the reference put that directory on sys.path and import
the modules by bare name (gpu/test_correctness.py:14-18); putting this directory
on sys.path instead gives them the HIP implementation.  Each module is a thin
re-export of polyhedral_amd's implementation, importable both ways.
"""
