"""gfx950 (MI355X) HIP kernels behind the reference's ``kernels.hip.*`` module API."""
