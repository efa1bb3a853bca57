"""MI355X-native page-sparse streaming attention (router, exact pages,
summary compensation, softmax-mass merge) on hand-written HIP kernels."""
