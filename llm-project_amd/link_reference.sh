#!/bin/bash
# link_reference.sh SRC DEST - build the reference's own `transformer` binary
# with its int8 LLaMA path served by libqllama.so (MI355X).
#
# Copies the reference checkout SRC to DEST (SRC itself is never modified), then:
#   llama.h   the LlamaKV typedef (llama.h:94-99) becomes #include "qllama.h",
#             which brings LlamaKV with its device handle, QTensor, QLlamaModel
#             and the quantized prototypes; the old quantized section
#             (llama.h:108-140) and #include "quant.h" (llama.h:17) go away
#   llama.c   the quantized section (llama.c:447-657) and the fp32 cache and
#             decode step (llama_kv_create, llama_kv_free, llama_decode_step,
#             llama.c:275-362) go away: the library serves both paths on the GPU
#   matrix.c  qacc_columns (matrix.c:370-374) goes away (the library exports it)
#   model.h   the KVCache typedef and the decode prototypes (model.h:124-136)
#             become #include "qgpt.h" (KVCache with its device handle)
#   model.c   gpt_kvcache_create / gpt_kvcache_free / gpt_decode_step
#             (model.c:437-523) go away: the library serves the GPT-2 decode
#   quant.c   is not compiled (the library exports its functions)
# and links -lqllama.  With GPU_SAMPLER=1 in the environment sampler.c is not
# compiled either: the library's sample_token / sample_argmax / rng_create /
# rng_uniform (same results, computed on the GPU) serve every caller.  The line numbers are those of the reference revision this
# library was built against; the script checks each anchor before editing.
set -euo pipefail
SRC=${1:?usage: link_reference.sh SRC DEST}
DEST=${2:?usage: link_reference.sh SRC DEST}
HERE=$(cd "$(dirname "$0")" && pwd)
INC=$(cd "$HERE/../include" && pwd)

check() {   # file line text: the anchor must be where the edit expects it
  if ! sed -n "$2p" "$DEST/$1" | grep -qF -- "$3"; then
    echo "link_reference.sh: $1:$2 is not '$3' (different reference revision?)" >&2
    exit 1
  fi
}

rm -rf "$DEST"
mkdir -p "$DEST"
cp -r "$SRC"/. "$DEST"/

check llama.h 17 '#include "quant.h"'
check llama.h 94 'typedef struct {'
check llama.h 99 '} LlamaKV;'
check llama.h 114 'typedef struct {'
check llama.h 140 'LlamaKV q_llama_kv_create(const QLlamaModel *m);'
check llama.c 275 'LlamaKV llama_kv_create(const LlamaModel *m) {'
check llama.c 290 'void llama_kv_free(LlamaKV *kv) {'
check llama.c 296 'void llama_decode_step(const LlamaModel *m, LlamaKV *kv, int token, Tensor *logits) {'
check llama.c 362 '}'
check llama.c 447 'static QLlamaBlock q_block_create('
check matrix.c 370 'void qacc_columns('
check model.h 124 'typedef struct {'
check model.h 129 '} KVCache;'
check model.h 136 'void gpt_decode_step(const GPT *m, KVCache *kv, int token, Tensor *logits);'
check model.c 437 'KVCache gpt_kvcache_create(const GPT *m) {'
check model.c 457 'void gpt_decode_step(const GPT *m, KVCache *kv, int token, Tensor *logits) {'
check model.c 523 '}'

# edits from the bottom up so the earlier line numbers stay valid
sed -i '108,140d; 94,99c #include "qllama.h"' "$DEST/llama.h"
sed -i '17d' "$DEST/llama.h"
sed -i '447,657d; 275,362d' "$DEST/llama.c"
sed -i '370,374d' "$DEST/matrix.c"
sed -i '124,136c #include "qgpt.h"' "$DEST/model.h"
sed -i '437,523d' "$DEST/model.c"

DROP='s/quant\.o//'
[ "${GPU_SAMPLER:-0}" = 1 ] && DROP='s/quant\.o//; s/sampler\.o//'
make -C "$DEST" transformer \
  CFLAGS="-std=c11 -O3 -march=native -Wall -pthread -I$INC" \
  OBJS="$(make -s -C "$DEST" -p -n 2>/dev/null | sed -n 's/^OBJS *= *//p' | head -1 | sed "$DROP")" \
  LDLIBS="-lm -pthread -L$HERE -lqllama -Wl,-rpath,$HERE"
echo "link_reference.sh: built $DEST/transformer against $HERE/libqllama.so"
