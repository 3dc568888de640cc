/*
 * dit_model.h — the reference's on-disk formats and model directory.
 *
 * Host readers of the three file formats the reference's DiT reads, and a
 * loader of a whole model directory in its layout onto the device, for
 * dit_forward_grid (dit_capi.h):
 *
 *   read_raw_f (dit_vk.cpp:38-45): int64 ndim, int64 shape[ndim], then
 *       prod(shape) float32 values.
 *   ncnn InnerProduct pair <base>.param / <base>.bin, as load_linear reads it
 *       (verify_dit.cpp:80-102): the InnerProduct line of .param carries
 *       0=num_output and 2=weight_data_size; .bin holds a 4-byte storage tag
 *       (0x01306B47: IEEE fp16 values follow; 0: float32), the weight
 *       [out][in], then, for layers with bias, out float32 values (no tag).
 *   load_win (dit_vk.cpp:74-93): 10 int64 [t, h, w, wt, wh, ww, nnt, nnh,
 *       nnw, nwin], nwin x 6 int64 slices [st, en, sh, eh, sw, ew], then the
 *       float32 frequency tables: vid_freq (sum f_w x 126) and txt_freq
 *       (nwin x txt_len x 126) back to back, split by txt_len.
 *
 * Host functions return 0 or -1 with a message in dit_host_last_error()
 * (per thread); buffers they return are freed with dit_free_host.
 */
#ifndef SEEDVR2_DIT_MODEL_H
#define SEEDVR2_DIT_MODEL_H

#include <stdint.h>

#include "dit_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* dit_host_last_error(void);
void dit_free_host(void* p);

/* read_raw_f: *data = malloc'd float32 values, *count of them; shape[0..ndim)
 * (room for 8 dimensions). */
int dit_read_raw_f(const char* path, float** data, int64_t* count, int64_t shape[8], int* ndim);

/* load_linear: *w = [n_out][n_in] float32 (fp16 storage widened exactly),
 * *b = [n_out] float32 if has_bias (else NULL). */
int dit_read_linear(const char* base, int has_bias, float** w, float** b, int* n_out, int* n_in);

/* load_win: header[10] as stored, *slices = nwin x 6 int32, the two
 * frequency tables and their float counts. */
int dit_read_win(const char* path, int txt_len, int64_t header[10], int32_t** slices, float** vid_freq,
                 int64_t* n_vid, float** txt_freq, int64_t* n_txt);

/* A model directory in the reference's layout (verify_dit.cpp:351-384,
 * dit_vk.cpp:157-177): vid_in_proj, txt_in, vid_out_proj, emb_proj_in,
 * emb_proj_hid, emb_proj_out (InnerProduct with bias); vid_out_norm_w.bin,
 * vid_out_ada_shift.bin, vid_out_ada_scale.bin (read_raw_f); per layer i
 * the branch b<i>_vid / b<i>_txt (i < mm_layers) or b<i>_all: _qkv, _out
 * (with bias), _mlp_in, _mlp_g, _mlp_out (InnerProduct) and _nq, _nk,
 * _attn_shift, _attn_scale, _attn_gate, _mlp_shift, _mlp_scale, _mlp_gate
 * (read_raw_f).  Linear weights go to the device as bf16 (RNE from their
 * stored values), vectors as float32; the reference checkpoint has
 * n_layers = 32, mm_layers = 10. */
typedef struct dit_model dit_model;
int dit_model_load(awa_ctx* ctx, const char* dir, int n_layers, int mm_layers, dit_model** out,
                   awa_stream_t stream);
/* n_layers, mm_layers and the SwiGLU width read from the files. */
int dit_model_info(const dit_model* m, int* n_layers, int* mm_layers, int* mlp);
/* dit_forward_grid with the model's weights. */
int dit_model_forward_grid(awa_ctx* ctx, const dit_model* m, const awa_geom* g_even,
                           const awa_geom* g_odd, int last_txt_vid_only, float eps, float t,
                           const float* d_grid, int T, int H, int W, const float* d_txt, int TXT,
                           float* d_x, float* d_out, awa_stream_t stream);
void dit_model_destroy(awa_ctx* ctx, dit_model* m);

/* The merged whole-model graph <g>.param / <g>.bin (export_dit_graph.py:
 * 47-258, loaded by DitVk's graph path, dit_graph.cpp:114-151): layer lines
 * Input, AdaCompose, InnerProduct (proj_vid_in, proj_txt_in, qkv_<i>_<v|t>,
 * out_, min_, mig_, mout_, outproj), RMSNorm (rn_fin with gamma), AWA
 * (awa_<i>), BinaryOp, Swish; the .bin is what each layer's load_model reads,
 * in layer order: AdaCompose's tagged vectors (per layer and flow attn_shift,
 * attn_scale, attn_gate, mlp_shift, mlp_scale, mlp_gate; then the output
 * layer's shift and scale, ada_compose.cpp:35-89), InnerProduct tagged weights
 * then raw bias, AWA four tagged 128-vectors (nq_v, nk_v, nq_t, nk_t,
 * awa_layer.cpp:38-52), the final RMSNorm's raw gamma.  Only a whole graph
 * (with the in_vid0 input and the output layer) is a model; block subgraphs
 * are refused.  The timestep MLP is not in the graph (the host runs it,
 * dit_graph.cpp:270): emb_proj_in/_hid/_out come from dir, the model
 * directory, as they do for DitVk::init.  mm_layers: the number of dual-branch
 * layers, -1 to take it from AdaCompose's 2= (required for a graph without
 * AdaCompose, whose ada vectors then also come from dir). */
int dit_model_load_graph(awa_ctx* ctx, const char* param, const char* bin, const char* dir, int mm_layers,
                         dit_model** out, awa_stream_t stream);
/* Host checks of a merged graph: its layer count, dual-branch count and the
 * number of distinct weights it indexes; and one weight by its model-directory
 * name (b3_vid_qkv, b12_all_nq, vid_out_norm_w, ...): linear weights as
 * [n_out][n_in] float32 with *b the bias or NULL, vectors with *n_out values
 * and *n_in = 0.  0, or -1 with dit_host_last_error(). */
int dit_graph_file_info(const char* param, const char* bin, int mm_layers, int* n_layers, int* mm_out,
                        int* n_weights);
int dit_read_graph_weight(const char* param, const char* bin, int mm_layers, const char* name, float** w,
                          float** b, int* n_out, int* n_in);

/* dit_model_forward_grid captured into one HIP graph per resolution (the
 * host orchestration of dit_graph.cpp:264-549 as a single replay).  The graph
 * runs on a private context of its own (its scratch cannot be reallocated
 * under it); creation runs the forward once eagerly on that context (leaving
 * its result in d_out), then captures it.  dit_graph_launch replays the whole
 * forward with the same arguments, reading the current contents of d_grid and
 * d_txt.  The model, the geometries and the buffers must outlive the graph;
 * launches of one graph must not overlap.  The capture stream must be a
 * created stream (the null stream cannot be captured). */
typedef struct dit_graph dit_graph;
int dit_graph_create(awa_ctx* ctx, const dit_model* m, const awa_geom* g_even, const awa_geom* g_odd,
                     int last_txt_vid_only, float eps, float t, const float* d_grid, int T, int H, int W,
                     const float* d_txt, int TXT, float* d_x, float* d_out, awa_stream_t stream,
                     dit_graph** out);
int dit_graph_launch(awa_ctx* ctx, dit_graph* g, awa_stream_t stream);
void dit_graph_destroy(dit_graph* g);

#ifdef __cplusplus
}
#endif
#endif
