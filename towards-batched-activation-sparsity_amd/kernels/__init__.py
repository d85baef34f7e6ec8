"""Import path of the reference's kernel module, served by the MI355X HIP implementation."""
