/* A C consumer of the h3attn ABI: compiled as C11 against include/h3attn.h
 * and linked with the built library, it calls the entry points that need no
 * GPU (version, argument validation, the workspace query) and prints what
 * they return, one "name value" pair per line. */
#include <stdio.h>
#include <string.h>

#include "h3attn.h"

int main(void) {
    printf("abi %d %d\n", h3a_abi_version(), H3A_ABI_VERSION);

    printf("null_args %d\n", h3a_attn_fwd(NULL, NULL));
    printf("null_args_message %d\n", strstr(h3a_last_error(), "args is NULL") != NULL);

    h3a_attn_args a;
    memset(&a, 0, sizeof(a));
    a.abi_version = H3A_ABI_VERSION;
    a.q = a.k = a.v = a.o = (void*)(uintptr_t)(1u << 20);
    a.batch = 1;
    a.heads = 4;
    a.seqlen_q = a.seqlen_k = 4096;
    a.head_dim = 128;
    const int64_t strides[3] = {4096 * 4 * 128, 4 * 128, 128};
    memcpy(a.q_stride, strides, sizeof(strides));
    memcpy(a.k_stride, strides, sizeof(strides));
    memcpy(a.v_stride, strides, sizeof(strides));
    memcpy(a.o_stride, strides, sizeof(strides));
    a.softmax_scale = 0.08838834764831845f;
    printf("workspace_ok %d\n", h3a_attn_fwd_workspace_size(&a) >= 0);

    a.head_dim = 64;
    printf("head_dim_64 %d\n", h3a_attn_fwd(&a, NULL));
    printf("head_dim_64_message %d\n", strstr(h3a_last_error(), "head_dim must be 128") != NULL);

    h3a_qknorm_rope_args r;
    memset(&r, 0, sizeof(r));
    r.abi_version = H3A_ABI_VERSION;
    r.batch = 1;
    r.seqlen = 8;
    r.heads = 2;
    r.head_dim = 128;
    r.rotary_dim = 7;
    printf("odd_rotary %d\n", h3a_qknorm_rope(&r, NULL));
    printf("odd_rotary_message %d\n",
           strstr(h3a_last_error(), "requires an even rotary dimension no wider than the head") != NULL);
    return 0;
}
