#!/bin/sh
# Adds the MI355X sampler binding and the sampling-parameter plumbing to an
# llm-rs checkout:  rust/apply.sh /path/to/llm-rs
# New files are copied in; the patches (zero-context unified diffs against
# llm-rs at the revision the sampler was built against) are applied with
# patch -p1.  Nothing is changed when any patch fails to apply.
set -eu
here=$(cd "$(dirname "$0")" && pwd)
dst=${1:?usage: apply.sh <llm-rs checkout>}
cd "$dst"
for p in "$here"/patches/*.patch; do
  patch -p1 --dry-run --silent < "$p" > /dev/null
done
for f in llm-kernel/src/hip_sampler.rs llm-kernel/build.rs llm-ffi/src/sampler.rs \
         llm-ffi/src/request_v2.rs; do
  if [ -e "$f" ]; then echo "apply.sh: $f exists already" >&2; exit 1; fi
done
for p in "$here"/patches/*.patch; do
  patch -p1 --silent < "$p"
done
cp "$here/llm-kernel/src/hip_sampler.rs" llm-kernel/src/
cp "$here/llm-kernel/build.rs" llm-kernel/
cp "$here/llm-ffi/src/sampler.rs" "$here/llm-ffi/src/request_v2.rs" llm-ffi/src/
echo "applied: build with --features llm-ffi/hip-sampler and LLMK_LIB_DIR=<dir of libllmk_sampler.so>"
