// Fusion compiler of the host runtime, re-targeted at gfx950: capture of a
// callback into a DAG (src/fusion_capture.c), plan building with the
// reference's inline-cost cut rule (src/fusion_plan.c:39-100, budget 32),
// HIP C++ code generation (replacing src/fusion_codegen.c's CUDA text),
// hipRTC compilation with a source-keyed module cache (src/fusion_cache.c)
// and replay, optionally through a captured HIP graph
// (src/fusion_execute.c:385-598).
//
// Generated kernels evaluate every fused root for a contiguous range of
// output elements.  When every leaf's address is an affine function of the
// output coordinates (elementwise ops, broadcasting, transposed / sliced
// leaves) the kernel walks the output four elements at a time: the
// coordinates are decoded once per group, unit-stride leaves load 16-byte
// vectors, zero-stride leaves load one scalar, and roots store 16-byte
// vectors.  Other graphs (reshaped intermediates) use per-node index
// functions with scalar accesses.  Node arithmetic matches the eager
// kernels exactly: operands converted to the node dtype (float for
// f16/bf16, rounded back after every node), no contraction (-ffp-contract=off),
// the same device libm.
#include "phpt_host.h"
#include "runtime.hpp"

#include <math.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

#include <algorithm>
#include <functional>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <unordered_map>

namespace phpt {

static constexpr int kKernelBudget = 32;  // FUSION_KERNEL_BUDGET, fusion_internal.h:18
static constexpr int kMaxNodes = 4096;

// ------------------------------------------------------------------- scope
struct Scope {
    std::vector<TensorP> recorded;
    std::vector<TensorP> inputs;
    bool compiling = false;
};
static thread_local Scope *t_scope = nullptr;

bool fusion_active() { return t_scope != nullptr; }

static TensorP record_node(std::shared_ptr<FusionNode> node, const int *shape, int ndims, int dtype)
{
    if (t_scope->recorded.size() >= (size_t)kMaxNodes) {
        set_invalid("Fusion graph exceeds %d nodes", kMaxNodes);
        return nullptr;
    }
    TensorP t = make_meta(shape, ndims, dtype);
    if (!t) return nullptr;
    t->node = node;
    t_scope->recorded.push_back(t);
    return t;
}

TensorP fusion_record(NodeKind kind, int op, std::vector<TensorP> inputs, const int *shape,
                      int ndims, int dtype)
{
    auto n = std::make_shared<FusionNode>();
    n->kind = kind;
    n->op = op;
    n->inputs = std::move(inputs);
    return record_node(n, shape, ndims, dtype);
}

TensorP fusion_record_scalar(const TensorP &a, const Scalar &s, int op, bool reverse, int dtype)
{
    auto n = std::make_shared<FusionNode>();
    n->kind = N_SCALAR;
    n->op = op;
    n->inputs = {a};
    n->scalar = s;
    n->reverse = reverse;
    return record_node(n, a->shape, a->ndims, dtype);
}

TensorP fusion_record_view(const TensorP &a, const int *shape, const size_t *strides, int ndims,
                           size_t offset)
{
    auto n = std::make_shared<FusionNode>();
    n->kind = N_VIEW;
    n->inputs = {a};
    for (int d = 0; d < ndims; d++) n->view_strides[d] = strides[d];
    n->view_offset = offset;
    return record_node(n, shape, ndims, a->dtype);
}

TensorP fusion_record_native(const NativeSpec &spec, std::vector<TensorP> inputs, const int *shape,
                             int ndims, int dtype)
{
    auto n = std::make_shared<FusionNode>();
    n->kind = N_NATIVE;
    n->native = spec;
    n->inputs = std::move(inputs);
    return record_node(n, shape, ndims, dtype);
}

// ------------------------------------------------------------------ plan
enum ItemKind { IT_CONST = 0, IT_INPUT, IT_ELEM, IT_NATIVE };

struct Item {
    TensorP t;
    int kind = IT_CONST;
    int input_index = -1;
    std::vector<int> args;
    int cost = 0;
    bool cut = false;       // materialized
    bool output = false;
    bool alias = false;     // view handed to a native step as a strided view (no copy)
    const char *reason = nullptr;
    int region = -1;        // dependent-output region (root item id), or -1
};

struct LeafMap {
    bool affine = false;
    long long offset = 0;              // element offset from the leaf base
    long long stride[kMaxDims] = {0};  // per output coordinate
};

struct Kernel {
    std::string name;
    bool dependent = false;       // a root evaluates another root of this kernel inline
    std::vector<int> roots;
    std::vector<int> leaves;      // items read through pointers
    int shape[kMaxDims] = {0};
    int ndims = 0;
    size_t total = 0;
    bool affine = false;          // vectorizable (affine leaf maps)
    std::vector<LeafMap> leaf_maps;
    std::vector<bool> leaf_vec;   // leaf read as 4-vectors in the vector kernel
    std::vector<bool> leaf_stream;  // leaf read once per element (nontemporal loads)
    pt_function_t fn_vec = nullptr;
    pt_function_t fn_scalar = nullptr;
};

struct Step {
    bool native = false;
    int kernel = -1;
    int item = -1;
};

// Row chain: plan steps that each work row by row on values of one row
// count (fused kernels whose reads of the chain's own values stay in the
// output's row, and native last-axis reductions of short fp32 rows), run by
// one generated kernel, one wave per row, at the position of the last
// member.  The plan's steps and their reported form are unchanged; only the
// number of launches drops.
struct RowChain {
    std::vector<int> members;     // step indices, in plan order
    long long rows = 0;
    std::vector<char> vec4;       // per member: a reduction whose rows are read as 4-element chunks
    std::string name;
    pt_function_t fn = nullptr;
};

struct Plan {
    std::vector<Item> items;
    std::vector<Kernel> kernels;
    std::vector<Step> steps;
    std::vector<int> outputs;        // item index per output
    std::vector<TensorP> input_examples;
    std::string source;
    pt_module_t module = nullptr;
    bool cache_hit = false;
    bool use_graph = false;
    bool graph_compatible = true;
    const char *incompatibility = nullptr;
    pt_graph_t graph = nullptr;
    std::vector<void *> graph_ptrs;  // pointers the captured graph was built with
    // FusionGraph::replay: the steps captured kReplayCopies times in a row
    // into one graph, for the buffers in batch_ptrs
    pt_graph_t batch_graph = nullptr;
    std::vector<void *> batch_ptrs;
    // buffer reuse: item index -> storage kept between runs
    std::unordered_map<int, std::shared_ptr<Storage>> cache;
    // statistics (FusionGraph::getStats, fusion.c:723-772)
    size_t executions = 0, graph_launches = 0, buffer_reuses = 0, tensor_allocations = 0;
    size_t synchronizations = 0;
    bool profiling = false;
    size_t profiled = 0;
    uint64_t bind_ns = 0, execute_ns = 0, collect_ns = 0;
    int pending = 0;  // submitted runAsync executions not yet waited for
    // scratch arena of the native steps inside the captured graph, sized by
    // the first (eager, measuring) run
    bool workspace_sized = false;
    size_t workspace_bytes = 0;
    std::shared_ptr<Storage> workspace;
    // indexed native steps (gather / scatterAdd): their invalid indices are
    // recorded in a device record that every execution clears and reads
    // back once (fusion_execute.c:630-645, 755-775); such plans neither
    // capture into a graph nor run asynchronously
    bool indexed = false;
    std::shared_ptr<Storage> index_record;
    // row chains (their kernels live in a module of their own, so that the
    // plan's generated source is what the steps alone produce)
    std::vector<RowChain> chains;
    std::vector<int> step_chain;     // per step: chain index, or -1
    std::string chain_source;
    pt_module_t chain_module = nullptr;
    size_t chain_fallbacks = 0;
};

static bool is_elementwise(const FusionNode &n)
{
    return n.kind == N_BINARY || n.kind == N_SCALAR || n.kind == N_UNARY || n.kind == N_CAST ||
           n.kind == N_WHERE || n.kind == N_VIEW;
}

static int collect(Plan &p, const TensorP &t, std::map<const Tensor *, int> &index)
{
    auto it = index.find(t.get());
    if (it != index.end()) return it->second;
    Item item;
    item.t = t;
    if (t->node && t->node->kind == N_INPUT) {
        item.kind = IT_INPUT;
        item.input_index = t->node->input_index;
    } else if (!t->node || t->storage) {
        item.kind = IT_CONST;
    } else {
        for (const TensorP &in : t->node->inputs) item.args.push_back(collect(p, in, index));
        item.kind = is_elementwise(*t->node) ? IT_ELEM : IT_NATIVE;
    }
    int id = (int)p.items.size();
    p.items.push_back(item);
    index[t.get()] = id;
    Item &me = p.items[id];
    // cost model (fusion_plan.c:39-100)
    if (me.kind == IT_ELEM) {
        const FusionNode &n = *t->node;
        int base = n.kind == N_UNARY ? 4 : n.kind == N_WHERE ? 3 : n.kind == N_VIEW ? 2
                 : n.op == PT_OP_POW ? 7 : 1;
        if (t->dtype == PT_FLOAT64) base *= 2;
        int cost = base;
        for (int a : me.args)
            if (p.items[a].kind == IT_ELEM && !p.items[a].cut) cost += p.items[a].cost;
        if (cost > kKernelBudget) {
            for (int a : me.args)
                if (p.items[a].kind == IT_ELEM && p.items[a].cost) {
                    p.items[a].cut = true;
                    p.items[a].reason = "expression-cost";
                }
            cost = base;
        }
        me.cost = cost;
    } else if (me.kind == IT_NATIVE) {
        me.cut = true;
        me.reason = "native";
        // GEMMs and (axis, or contiguous global) reductions read views of
        // materialized values in place, as the reference's layout aliases do
        // (fusion_plan.c:462-486); other native steps take a materialized
        // operand
        const NativeSpec &ns = t->node->native;
        const bool aliasing = ns.kind == NAT_MATMUL || ns.kind == NAT_REDUCE || ns.kind == NAT_ARG_REDUCE;
        const bool global = (ns.kind == NAT_REDUCE || ns.kind == NAT_ARG_REDUCE) && ns.axis == kGlobalAxis;
        for (int a : me.args) {
            Item &ai = p.items[a];
            if (ai.kind != IT_ELEM) continue;
            bool view = !ai.cut && ai.t->node->kind == N_VIEW;
            if (view && global) {
                size_t cs[kMaxDims];
                contiguous_strides(ai.t->shape, ai.t->ndims, cs);
                for (int d = 0; d < ai.t->ndims; d++)
                    if (ai.t->shape[d] != 1 && ai.t->node->view_strides[d] != cs[d]) view = false;
            }
            if (!aliasing || !view) {
                ai.cut = true;
                if (!ai.reason) ai.reason = "native-input";
                continue;
            }
            // a chain of views over a value reaches the native step as a
            // strided view of that value: only its base is materialized
            ai.alias = true;
            int b = a;
            while (p.items[b].kind == IT_ELEM && !p.items[b].cut && p.items[b].t->node->kind == N_VIEW)
                b = p.items[b].args[0];
            if (p.items[b].kind == IT_ELEM && !p.items[b].cut) {
                p.items[b].cut = true;
                p.items[b].reason = "native-input";
            }
        }
    }
    return id;
}

// Steps that item `id` reads directly: cut elementwise items and native
// items reached through uncut elementwise items (not past another step).
static void direct_deps(const Plan &p, int id, std::vector<int> &out)
{
    std::vector<char> seen(p.items.size(), 0);
    std::function<void(int)> walk = [&](int x) {
        if (seen[x]) return;
        seen[x] = 1;
        const Item &it = p.items[x];
        if (it.kind == IT_NATIVE || (it.kind == IT_ELEM && it.cut)) {
            out.push_back(x);
            return;
        }
        if (it.kind != IT_ELEM) return;
        for (int a : it.args) walk(a);
    };
    for (int a : p.items[id].args) walk(a);
}

// ------------------------------------------------------------ leaf maps
// Affine map of item `id` evaluated at output coordinates: element offset
// (relative to the leaf's base pointer) = off + sum c_d * st[d] over the
// kernel's output dims.  `st` expresses the item's *logical* coordinates
// in output coordinates, then leaf strides are applied.
struct CoordMap {
    // item coordinate k = sum over output dims d of coef[k][d] * c_d + base[k]
    int nd_item = 0;
    long long coef[kMaxDims][kMaxDims];
    long long base[kMaxDims];
};

static CoordMap identity_map(int nd)
{
    CoordMap m;
    m.nd_item = nd;
    for (int k = 0; k < nd; k++) {
        for (int d = 0; d < nd; d++) m.coef[k][d] = k == d ? 1 : 0;
        m.base[k] = 0;
    }
    return m;
}

// operand of a broadcasting node: align trailing dims, extent-1 dims pinned to 0
static CoordMap broadcast_child(const CoordMap &parent, const Tensor &parent_t, const Tensor &child, int nd_out)
{
    CoordMap m;
    m.nd_item = child.ndims;
    int off = parent_t.ndims - child.ndims;
    for (int k = 0; k < child.ndims; k++) {
        int pk = k + off;
        for (int d = 0; d < nd_out; d++) m.coef[k][d] = child.shape[k] == 1 ? 0 : parent.coef[pk][d];
        m.base[k] = child.shape[k] == 1 ? 0 : parent.base[pk];
    }
    return m;
}

struct Codegen {
    Plan &p;
    Kernel &k;
    std::ostringstream &os;
    std::map<int, int> leaf_slot;  // item -> leaf parameter index
};

static const char *ctype(int dt)
{
    switch (dt) {
    case PT_FLOAT32: case PT_FLOAT16: case PT_BFLOAT16: return "float";
    case PT_FLOAT64: return "double";
    case PT_INT8: return "signed char";
    case PT_INT16: return "short";
    case PT_INT32: return "int";
    case PT_INT64: return "long long";
    case PT_UINT8: return "unsigned char";
    case PT_UINT16: return "unsigned short";
    case PT_UINT32: return "unsigned int";
    case PT_UINT64: return "unsigned long long";
    case PT_BOOL: return "bool";
    default: return "float";
    }
}

static const char *storage_type(int dt)
{
    switch (dt) {
    case PT_FLOAT16: case PT_BFLOAT16: return "unsigned short";
    case PT_BOOL: return "unsigned char";
    default: return ctype(dt);
    }
}

// Read of raw storage value `expr` of dtype dt as its compute type.
static std::string load_conv(int dt, const std::string &expr)
{
    if (dt == PT_FLOAT16) return "pt_h2f(" + expr + ")";
    if (dt == PT_BFLOAT16) return "pt_b2f(" + expr + ")";
    if (dt == PT_BOOL) return "(" + expr + "!=0)";
    return expr;
}

// Conversion of a compute-type value to storage of dtype dt.
static std::string store_conv(int dt, const std::string &expr)
{
    if (dt == PT_FLOAT16) return "pt_f2h(" + expr + ")";
    if (dt == PT_BFLOAT16) return "pt_f2b(" + expr + ")";
    if (dt == PT_BOOL) return "(unsigned char)((" + expr + ")!=0)";
    return expr;
}

static std::string scalar_literal(const Scalar &s)
{
    char buf[96];
    switch (s.dtype) {
    case PT_FLOAT64: {
        uint64_t bits;
        memcpy(&bits, &s.f, 8);
        snprintf(buf, sizeof(buf), "__longlong_as_double(0x%llxLL)", (unsigned long long)bits);
        break;
    }
    case PT_FLOAT32: case PT_FLOAT16: case PT_BFLOAT16: {
        float f = (float)s.f;
        uint32_t bits;
        memcpy(&bits, &f, 4);
        snprintf(buf, sizeof(buf), "__uint_as_float(0x%xu)", bits);
        break;
    }
    case PT_BOOL: snprintf(buf, sizeof(buf), "%s", s.u ? "true" : "false"); break;
    case PT_UINT8: case PT_UINT16: case PT_UINT32: case PT_UINT64:
        snprintf(buf, sizeof(buf), "%lluULL", (unsigned long long)s.u);
        break;
    default: snprintf(buf, sizeof(buf), "(long long)%lldLL", (long long)s.i); break;
    }
    return buf;
}

static const char *math_name(int op)
{
    switch (op) {
    case PT_OP_EXP: return "exp";
    case PT_OP_EXPM1: return "expm1";
    case PT_OP_EXP2: return "exp2";
    case PT_OP_LOG: return "log";
    case PT_OP_LOG1P: return "log1p";
    case PT_OP_LOG2: return "log2";
    case PT_OP_LOG10: return "log10";
    case PT_OP_SQRT: return "sqrt";
    case PT_OP_SIN: return "sin";
    case PT_OP_COS: return "cos";
    case PT_OP_TAN: return "tan";
    case PT_OP_ASIN: return "asin";
    case PT_OP_ACOS: return "acos";
    case PT_OP_ATAN: return "atan";
    case PT_OP_SINH: return "sinh";
    case PT_OP_COSH: return "cosh";
    case PT_OP_TANH: return "tanh";
    case PT_OP_FLOOR: return "floor";
    case PT_OP_CEIL: return "ceil";
    case PT_OP_ROUND: return "round";
    default: return nullptr;
    }
}

// Expression of node `id` (compute type of its dtype) given operand
// expressions; mirrors the eager kernels' bin_op / unary rules.
static std::string node_expr(const Plan &p, int id, const std::vector<std::string> &a)
{
    const Item &it = p.items[id];
    const Tensor &t = *it.t;
    const FusionNode &n = *t.node;
    std::string T = ctype(t.dtype);
    bool int_out = !is_floating(t.dtype) && t.dtype != PT_BOOL;
    auto cast = [&](const std::string &e) { return "static_cast<" + T + ">(" + e + ")"; };
    std::string r;
    switch (n.kind) {
    case N_CAST:
        if (t.dtype == PT_BOOL) r = "(" + a[0] + "!=0)";
        else r = cast(a[0]);
        break;
    case N_VIEW: r = a[0]; break;
    case N_WHERE: r = "((" + a[0] + ")!=0?" + cast(a[1]) + ":" + cast(a[2]) + ")"; break;
    case N_UNARY: {
        std::string x = cast(a[0]);
        if (n.op == PT_OP_NEG) r = "(-" + x + ")";
        else if (n.op == PT_OP_ABS) r = "(" + x + "<0?-" + x + ":" + x + ")";
        else if (int_out && (n.op == PT_OP_FLOOR || n.op == PT_OP_CEIL || n.op == PT_OP_ROUND)) r = x;
        else if (int_out || t.dtype == PT_BOOL)
            r = cast(std::string(math_name(n.op)) + "f(static_cast<float>(" + x + "))");
        else
            r = std::string(math_name(n.op)) + (t.dtype == PT_FLOAT64 ? "" : "f") + "(" + x + ")";
        break;
    }
    case N_BINARY:
    case N_SCALAR: {
        std::string x, y;
        if (n.kind == N_BINARY) {
            x = cast(a[0]);
            y = cast(a[1]);
        } else {
            std::string sv = cast(scalar_literal(n.scalar));
            x = n.reverse ? sv : cast(a[0]);
            y = n.reverse ? cast(a[0]) : sv;
        }
        switch (n.op) {
        case PT_OP_ADD: r = "(" + x + "+" + y + ")"; break;
        case PT_OP_SUB: r = "(" + x + "-" + y + ")"; break;
        case PT_OP_MUL: r = "(" + x + "*" + y + ")"; break;
        case PT_OP_DIV:
            r = int_out ? "(" + y + "==0?" + cast("0") + ":" + x + "/" + y + ")" : "(" + x + "/" + y + ")";
            break;
        case PT_OP_POW: r = (int_out ? "pt_powi(" : "pt_pow(") + x + "," + y + ")"; break;
        case PT_OP_MAXIMUM: r = "(" + x + ">" + y + "?" + x + ":" + y + ")"; break;
        case PT_OP_MINIMUM: r = "(" + x + "<" + y + "?" + x + ":" + y + ")"; break;
        case PT_OP_GT: r = "(" + x + ">" + y + "?" + cast("1") + ":" + cast("0") + ")"; break;
        case PT_OP_LT: r = "(" + x + "<" + y + "?" + cast("1") + ":" + cast("0") + ")"; break;
        case PT_OP_EQ: r = "(" + x + "==" + y + "?" + cast("1") + ":" + cast("0") + ")"; break;
        case PT_OP_NE: r = "(" + x + "!=" + y + "?" + cast("1") + ":" + cast("0") + ")"; break;
        case PT_OP_GE: r = "(" + x + ">=" + y + "?" + cast("1") + ":" + cast("0") + ")"; break;
        case PT_OP_LE: r = "(" + x + "<=" + y + "?" + cast("1") + ":" + cast("0") + ")"; break;
        default: r = x; break;
        }
        break;
    }
    default: r = "0"; break;
    }
    // low-precision nodes round after every op (eager kernels store them)
    if (t.dtype == PT_FLOAT16) r = "pt_h2f(pt_f2h(" + r + "))";
    else if (t.dtype == PT_BFLOAT16) r = "pt_b2f(pt_f2b(" + r + "))";
    return r;
}

static bool is_leaf(const Plan &p, const Kernel &k, int id)
{
    const Item &it = p.items[id];
    if (it.kind != IT_ELEM) return true;
    if (!it.cut) return false;
    return std::find(k.roots.begin(), k.roots.end(), id) == k.roots.end();
}

// Gather leaves of a kernel and decide whether every leaf map is affine.
static void gather(const Plan &p, Kernel &k, int id, const CoordMap &cm, bool &affine,
                   std::vector<std::pair<int, CoordMap>> &uses)
{
    const Item &it = p.items[id];
    if (is_leaf(p, k, id)) {
        uses.push_back({id, cm});
        if (std::find(k.leaves.begin(), k.leaves.end(), id) == k.leaves.end()) k.leaves.push_back(id);
        return;
    }
    const Tensor &t = *it.t;
    const FusionNode &n = *t.node;
    if (n.kind == N_VIEW) {
        // source linear index = off + sum coord_d * view_stride_d; affine in
        // the source's coordinates only when the source is 1-D or the view
        // strides decompose; keep the general path for these.
        affine = false;
        CoordMap dummy = identity_map(p.items[it.args[0]].t->ndims);
        gather(p, k, it.args[0], dummy, affine, uses);
        return;
    }
    for (int a : it.args) {
        const Tensor &c = *p.items[a].t;
        gather(p, k, a, broadcast_child(cm, t, c, k.ndims), affine, uses);
    }
}

// ------------------------------------------------------ code generation
static void emit_prelude(std::ostringstream &os)
{
    // hipRTC provides the HIP device builtins and vector types itself
    os << "typedef unsigned int pt_u4 __attribute__((ext_vector_type(4)));\n"
          "typedef unsigned int pt_u2 __attribute__((ext_vector_type(2)));\n"
          "__device__ __forceinline__ float pt_b2f(unsigned short b){return __uint_as_float(((unsigned)b)<<16);}\n"
          "__device__ __forceinline__ unsigned short pt_f2b(float f){unsigned u=__float_as_uint(f);"
          "if((u&0x7f800000u)==0x7f800000u&&(u&0x7fffffu))return (unsigned short)((u>>16)|0x40u);"
          "return (unsigned short)((u+0x7fffu+((u>>16)&1u))>>16);}\n"
          "__device__ __forceinline__ float pt_h2f(unsigned short h){return (float)__builtin_bit_cast(_Float16,h);}\n"
          "__device__ __forceinline__ unsigned short pt_f2h(float f){unsigned u=__float_as_uint(f);"
          "if((u&0x7f800000u)==0x7f800000u&&(u&0x7fffffu)){unsigned p=(u&0x7fffffu)>>13;if(!p)p=1;"
          "return (unsigned short)(((u>>16)&0x8000u)|0x7c00u|p);}return __builtin_bit_cast(unsigned short,(_Float16)f);}\n"
          "template<typename T>__device__ __forceinline__ T pt_ipow(T b,int e){T r=(T)1;while(e>0){if(e&1)r=r*b;b=b*b;e>>=1;}return r;}\n"
          "__device__ __forceinline__ float pt_pow(float a,float b){if(b==floorf(b)){int e=(int)b;"
          "if(e==0)return 1.0f;if(e==1)return a;if(e==2)return a*a;if(e==3)return a*a*a;"
          "if(e<0)return 1.0f/pt_ipow(a,-e);return pt_ipow(a,e);}return powf(a,b);}\n"
          "__device__ __forceinline__ double pt_pow(double a,double b){if(b==floor(b)){int e=(int)b;"
          "if(e==0)return 1.0;if(e==1)return a;if(e==2)return a*a;if(e==3)return a*a*a;"
          "if(e<0)return 1.0/pt_ipow(a,-e);return pt_ipow(a,e);}return pow(a,b);}\n"
          "template<typename T>__device__ __forceinline__ T pt_powi(T a,T b){int e=(int)b;"
          "if(e==0)return (T)1;if(e==1)return a;if(e==2)return a*a;if(e==3)return a*a*a;"
          "if(e<0)return (T)0;return pt_ipow(a,e);}\n";
}

// General path: one device function per node, evaluated at the node's own
// linear index (as the reference codegen does), scalar accesses.  The node
// functions of kernel `k` are named <k.name>_n<item> and take the kernel's
// leaf pointers p0.. in leaf order, then the index.
static void emit_node_functions(Plan &p, Kernel &k, std::ostringstream &os)
{
    std::vector<char> emitted(p.items.size(), 0);
    std::string params;
    for (size_t l = 0; l < k.leaves.size(); l++) params += "const void* __restrict__ p" + std::to_string(l) + ",";
    std::string args;
    for (size_t l = 0; l < k.leaves.size(); l++) args += "p" + std::to_string(l) + ",";
    std::function<void(int)> emit = [&](int id) {
        if (emitted[id]) return;
        emitted[id] = 1;
        const Item &it = p.items[id];
        const Tensor &t = *it.t;
        std::string fname = k.name + "_n" + std::to_string(id);
        bool leaf = is_leaf(p, k, id);
        if (!leaf)
            for (int a : it.args) emit(a);
        os << "__device__ __forceinline__ " << ctype(t.dtype) << " " << fname << "(" << params
           << "unsigned long long i){\n";
        if (leaf) {
            int slot = (int)(std::find(k.leaves.begin(), k.leaves.end(), id) - k.leaves.begin());
            // leaves read with their own strides (constants, inputs) or
            // contiguously (materialized buffers)
            bool own = it.kind == IT_CONST || it.kind == IT_INPUT;
            const Tensor &src = (it.kind == IT_INPUT) ? *p.input_examples[it.input_index] : t;
            os << "unsigned long long o=0;\n";
            unsigned long long div = 1;
            for (int d = t.ndims - 1; d >= 0; d--) {
                unsigned long long st = own ? (unsigned long long)src.strides[d] : div;
                if (t.shape[d] > 1)
                    os << "o+=((i/" << div << "ULL)%" << t.shape[d] << "ULL)*" << st << "ULL;\n";
                div *= (unsigned long long)(t.shape[d] ? t.shape[d] : 1);
            }
            os << "return " << load_conv(t.dtype, std::string("static_cast<const ") + storage_type(t.dtype) +
                                                       "*>(p" + std::to_string(slot) + ")[o]")
               << ";}\n";
            return;
        }
        const FusionNode &n = *t.node;
        std::vector<std::string> ops;
        int c = 0;
        for (int a : it.args) {
            const Tensor &ct = *p.items[a].t;
            std::string var = "i" + std::to_string(c++);
            if (n.kind == N_VIEW) {
                os << "unsigned long long " << var << "=" << n.view_offset << "ULL;\n";
                unsigned long long div = 1;
                for (int d = t.ndims - 1; d >= 0; d--) {
                    if (t.shape[d] > 1)
                        os << var << "+=((i/" << div << "ULL)%" << t.shape[d] << "ULL)*" << n.view_strides[d]
                           << "ULL;\n";
                    div *= (unsigned long long)(t.shape[d] ? t.shape[d] : 1);
                }
            } else {
                // broadcast projection of the output index onto the operand
                os << "unsigned long long " << var << "=0;\n";
                unsigned long long div = 1, st = 1;
                int off = t.ndims - ct.ndims;
                for (int d = t.ndims - 1; d >= 0; d--) {
                    int cd = d - off;
                    if (cd >= 0) {
                        if (ct.shape[cd] != 1 && t.shape[d] > 1)
                            os << var << "+=((i/" << div << "ULL)%" << t.shape[d] << "ULL)*" << st << "ULL;\n";
                        st *= (unsigned long long)(ct.shape[cd] ? ct.shape[cd] : 1);
                    }
                    div *= (unsigned long long)(t.shape[d] ? t.shape[d] : 1);
                }
            }
            os << ctype(ct.dtype) << " v" << (c - 1) << "=" << k.name << "_n" << a << "(" << args << var << ");\n";
            ops.push_back("v" + std::to_string(c - 1));
        }
        os << "return " << node_expr(p, id, ops) << ";}\n";
    };
    for (int r : k.roots) emit(r);
}

static void emit_general(Plan &p, Kernel &k, std::ostringstream &os)
{
    emit_node_functions(p, k, os);
    std::string params;
    for (size_t l = 0; l < k.leaves.size(); l++) params += "const void* __restrict__ p" + std::to_string(l) + ",";
    std::string args;
    for (size_t l = 0; l < k.leaves.size(); l++) args += "p" + std::to_string(l) + ",";
    os << "extern \"C\" __global__ void " << k.name << "_s(" << params;
    for (size_t r = 0; r < k.roots.size(); r++) os << (r ? "," : "") << "void* __restrict__ out" << r;
    os << "){for(unsigned long long i=(unsigned long long)blockIdx.x*blockDim.x+threadIdx.x;i<" << k.total
       << "ULL;i+=(unsigned long long)blockDim.x*gridDim.x){\n";
    for (size_t r = 0; r < k.roots.size(); r++) {
        int id = k.roots[r];
        const Tensor &t = *p.items[id].t;
        os << "static_cast<" << storage_type(t.dtype) << "*>(out" << r << ")[i]="
           << store_conv(t.dtype, k.name + "_n" + std::to_string(id) + "(" + args + "i)") << ";\n";
    }
    os << "}}\n";
}

// Vector path: coordinates decoded once per group of 4 output elements.
// Leaves that stream (read once per output element) and the outputs use
// nontemporal 16-byte / 8-byte accesses so that they do not displace the
// broadcast operands from L2 and the Infinity Cache.
static std::string bits_to_ctype(int dt, const std::string &raw)
{
    switch (dt) {
    case PT_FLOAT32: return "__uint_as_float(" + raw + ")";
    case PT_FLOAT16: return "pt_h2f((unsigned short)(" + raw + "))";
    case PT_BFLOAT16: return "pt_b2f((unsigned short)(" + raw + "))";
    default: return "static_cast<" + std::string(ctype(dt)) + ">(" + raw + ")";
    }
}

static void emit_vector(Plan &p, Kernel &k, std::ostringstream &os)
{
    std::string params;
    for (size_t l = 0; l < k.leaves.size(); l++) params += "const void* __restrict__ p" + std::to_string(l) + ",";
    os << "extern \"C\" __global__ __launch_bounds__(256) void " << k.name << "_v(" << params;
    for (size_t r = 0; r < k.roots.size(); r++) os << (r ? "," : "") << "void* __restrict__ out" << r;
    const int nd = k.ndims;
    // 32-bit index arithmetic (division by the constant extents becomes a
    // multiply-high) when the element count and every leaf offset fit
    bool i32 = k.total < (1ULL << 32);
    for (const LeafMap &m : k.leaf_maps) {
        long long reach = m.offset;
        if (m.offset < 0) i32 = false;
        for (int d = 0; d < nd; d++) {
            if (m.stride[d] < 0) i32 = false;
            reach += (long long)(k.shape[d] - 1) * m.stride[d];
        }
        if (reach >= (1LL << 32)) i32 = false;
    }
    const std::string IT = i32 ? "unsigned int" : "unsigned long long", SUF = i32 ? "U" : "ULL";
    os << "){\nconst " << IT << " n4=" << k.total / 4 << SUF << ";\n"
       << "for(" << IT << " g=(" << IT << ")blockIdx.x*blockDim.x+threadIdx.x;g<n4;"
       << "g+=(" << IT << ")blockDim.x*gridDim.x){\n"
       << "const " << IT << " i0=g*4" << SUF << ";\n";
    // coordinates of element i0
    unsigned long long div = 1;
    for (int d = nd - 1; d >= 0; d--) {
        os << "const " << IT << " c" << d << "=(i0/" << div << SUF << ")%" << k.shape[d] << SUF << ";\n";
        div *= (unsigned long long)k.shape[d];
    }
    const char *f[4] = {"x", "y", "z", "w"};
    // leaf loads: L<slot>_<j>
    for (size_t l = 0; l < k.leaves.size(); l++) {
        const LeafMap &m = k.leaf_maps[l];
        int id = k.leaves[l];
        const Tensor &t = *p.items[id].t;
        std::string st = storage_type(t.dtype);
        std::string L = "L" + std::to_string(l);
        os << "const " << IT << " o" << l << "=" << m.offset << SUF;
        for (int d = 0; d < nd; d++)
            if (m.stride[d]) os << "+c" << d << "*" << m.stride[d] << SUF;
        os << ";\n";
        std::string base = "static_cast<const " + st + "*>(p" + std::to_string(l) + ")";
        std::string at = base + "+o" + std::to_string(l);
        long long inner = nd ? m.stride[nd - 1] : 0;
        size_t es = dtype_size(t.dtype);
        bool nt = k.leaf_stream[l];
        if (inner == 0) {
            os << "const " << ctype(t.dtype) << " " << L << "=" << load_conv(t.dtype, base + "[o" + std::to_string(l) + "]")
               << ";\n";
            for (int j = 0; j < 4; j++)
                os << "const " << ctype(t.dtype) << " " << L << "_" << j << "=" << L << ";\n";
        } else if (inner == 1 && k.leaf_vec[l] && es == 4) {
            std::string ptr = "reinterpret_cast<const pt_u4*>(" + at + ")";
            os << "const pt_u4 R" << l << "=" << (nt ? "__builtin_nontemporal_load(" + ptr + ")" : "*" + ptr) << ";\n";
            for (int j = 0; j < 4; j++)
                os << "const " << ctype(t.dtype) << " " << L << "_" << j << "="
                   << bits_to_ctype(t.dtype, "R" + std::to_string(l) + "." + f[j]) << ";\n";
        } else if (inner == 1 && k.leaf_vec[l] && es == 2) {
            std::string ptr = "reinterpret_cast<const pt_u2*>(" + at + ")";
            os << "const pt_u2 R" << l << "=" << (nt ? "__builtin_nontemporal_load(" + ptr + ")" : "*" + ptr) << ";\n";
            for (int j = 0; j < 4; j++) {
                std::string raw = "(R" + std::to_string(l) + "." + (j < 2 ? "x" : "y") + (j % 2 ? ">>16" : "&0xffffu") + ")";
                os << "const " << ctype(t.dtype) << " " << L << "_" << j << "=" << bits_to_ctype(t.dtype, raw) << ";\n";
            }
        } else {
            for (int j = 0; j < 4; j++)
                os << "const " << ctype(t.dtype) << " " << L << "_" << j << "="
                   << load_conv(t.dtype, base + "[o" + std::to_string(l) + "+" + std::to_string(j * inner) + SUF + "]")
                   << ";\n";
        }
    }
    // per element j: evaluate the roots' expression trees
    for (int j = 0; j < 4; j++) {
        std::map<int, std::string> val;
        std::function<std::string(int)> ev = [&](int id) -> std::string {
            auto it = val.find(id);
            if (it != val.end()) return it->second;
            if (is_leaf(p, k, id)) {
                int slot = (int)(std::find(k.leaves.begin(), k.leaves.end(), id) - k.leaves.begin());
                return val[id] = "L" + std::to_string(slot) + "_" + std::to_string(j);
            }
            std::vector<std::string> ops;
            for (int a : p.items[id].args) ops.push_back(ev(a));
            std::string name = "e" + std::to_string(id) + "_" + std::to_string(j);
            os << "const " << ctype(p.items[id].t->dtype) << " " << name << "=" << node_expr(p, id, ops) << ";\n";
            return val[id] = name;
        };
        for (int r : k.roots) ev(r);
        for (size_t r = 0; r < k.roots.size(); r++) {
            int id = k.roots[r];
            os << "const " << ctype(p.items[id].t->dtype) << " r" << r << "_" << j << "=" << val[id] << ";\n";
        }
    }
    // outputs are contiguous and 16-byte aligned (checked at launch)
    for (size_t r = 0; r < k.roots.size(); r++) {
        const Tensor &t = *p.items[k.roots[r]].t;
        std::string st = storage_type(t.dtype);
        std::string rv = "r" + std::to_string(r) + "_";
        std::string out = "static_cast<" + st + "*>(out" + std::to_string(r) + ")+i0";
        size_t es = dtype_size(t.dtype);
        auto bits = [&](int j) {
            std::string v = rv + std::to_string(j);
            if (t.dtype == PT_FLOAT32) return "__float_as_uint(" + v + ")";
            if (es == 4) return "static_cast<unsigned int>(" + v + ")";
            return "(unsigned int)(unsigned short)(" + store_conv(t.dtype, v) + ")";
        };
        if (es == 4) {
            os << "__builtin_nontemporal_store((pt_u4){" << bits(0) << "," << bits(1) << "," << bits(2) << ","
               << bits(3) << "},reinterpret_cast<pt_u4*>(" << out << "));\n";
        } else if (es == 2) {
            os << "__builtin_nontemporal_store((pt_u2){" << bits(0) << "|(" << bits(1) << "<<16)," << bits(2) << "|("
               << bits(3) << "<<16)},reinterpret_cast<pt_u2*>(" << out << "));\n";
        } else {
            for (int j = 0; j < 4; j++)
                os << "static_cast<" << st << "*>(out" << r << ")[i0+" << j << "]="
                   << store_conv(t.dtype, rv + std::to_string(j)) << ";\n";
        }
    }
    os << "}}\n";
}

// ------------------------------------------------------------ module cache
struct ModuleCache {
    std::mutex mu;
    std::unordered_map<std::string, pt_module_t> modules;
    std::vector<std::string> order;
    size_t hits = 0, misses = 0, evictions = 0, compilations = 0;
    size_t bytes = 0;  // source text held as keys
};
static ModuleCache g_cache;
// fusion_cache.c: a 16-entry, 16 MiB LRU (FUSION_CACHE_ENTRIES / _BYTES)
static const size_t kCacheEntries = 16;
static const size_t kCacheBytes = 16u << 20;

static pt_module_t load_module(const std::string &src, bool &hit)
{
    std::lock_guard<std::mutex> lock(g_cache.mu);
    auto it = g_cache.modules.find(src);
    if (it != g_cache.modules.end()) {
        hit = true;
        g_cache.hits++;
        auto pos = std::find(g_cache.order.begin(), g_cache.order.end(), src);
        if (pos != g_cache.order.end()) {
            g_cache.order.erase(pos);
            g_cache.order.push_back(src);
        }
        return it->second;
    }
    hit = false;
    g_cache.misses++;
    pt_module_t m = nullptr;
    static char log[8192];
    if (!check_status(pt_rtc_compile(src.c_str(), "fusion.hip", &m, log, sizeof(log)), "Fusion compilation failed"))
        return nullptr;
    // modules stay loaded while plans may use them; eviction only drops
    // the cache entry (compiled graphs keep their module handle)
    g_cache.compilations++;
    g_cache.modules[src] = m;
    g_cache.order.push_back(src);
    g_cache.bytes += src.size();
    while (g_cache.order.size() > kCacheEntries ||
           (g_cache.bytes > kCacheBytes && g_cache.order.size() > 1)) {
        g_cache.bytes -= g_cache.order.front().size();
        g_cache.modules.erase(g_cache.order.front());
        g_cache.order.erase(g_cache.order.begin());
        g_cache.evictions++;
    }
    return m;
}

// ------------------------------------------------------ output regions
// Dependent-output regions (the rule of the reference's
// fusion_output_regions, fusion_plan.c:250-397).  An output is grown into a
// region of same-shape floating elementwise items: the region takes the
// output's compatible ancestors, then, output by output in item order and
// until nothing changes, every other output that reaches the region through
// compatible items, together with that output's compatible ancestors, while
// the members' operation costs sum to at most kRegionBudget and at most four
// outputs are members.  The region stands when it holds two or more outputs,
// at most four values leave it (member outputs, and members read by other
// items), and no path leaves it and comes back (a member reading an outside
// item that depends on a member).  One kernel then evaluates the region;
// only the values that leave it are materialized.
//
// Items are stored after their arguments, so each reachability question is
// one sweep over the item order: backward for a set of ancestors, forward for
// "reaches the region".
static constexpr int kRegionBudget = 128;

static bool region_member_kind(const Plan &p, int id, int shape_of)
{
    const Item &it = p.items[id];
    if (it.kind != IT_ELEM || it.region >= 0 || it.alias) return false;
    const FusionNode &n = *it.t->node;
    if (n.kind != N_BINARY && n.kind != N_SCALAR && n.kind != N_UNARY && n.kind != N_WHERE &&
        n.kind != N_CAST)
        return false;
    const Tensor &t = *it.t, &r = *p.items[shape_of].t;
    if (t.dtype != PT_FLOAT32 && t.dtype != PT_FLOAT64 && t.dtype != PT_BOOL) return false;
    return t.ndims == r.ndims && std::equal(t.shape, t.shape + t.ndims, r.shape);
}

// operation cost of one member (the reference's region cost table)
static int region_op_cost(const Item &it)
{
    const FusionNode &n = *it.t->node;
    int c = n.kind == N_UNARY ? 4 : n.kind == N_WHERE ? 3 : n.op == PT_OP_POW ? 7 : 1;
    return it.t->dtype == PT_FLOAT64 ? 2 * c : c;
}

class RegionBuilder {
public:
    RegionBuilder(const Plan &plan, int root) : p_(plan), n_((int)plan.items.size()), compat_(n_, 0)
    {
        for (int i = 0; i < n_; i++) compat_[i] = region_member_kind(p_, i, root);
    }

    // Adds `start` and its compatible ancestors that `set` lacks (an item in
    // `set`, or one that cannot join, is not looked through); false when the
    // cost then exceeds the budget.
    bool absorb(int start, std::vector<char> &set, int &cost) const
    {
        std::vector<char> wanted(n_, 0);
        wanted[start] = 1;
        for (int x = start; x >= 0; x--) {
            if (!wanted[x] || set[x] || !compat_[x]) continue;
            set[x] = 1;
            cost += region_op_cost(p_.items[x]);
            for (int a : p_.items[x].args) wanted[a] = 1;
        }
        return cost <= kRegionBudget;
    }

    // r[x]: x is in `set` or one of its arguments reaches it; with
    // `through_compatible`, only items that can join pass the reach on
    std::vector<char> reaching(const std::vector<char> &set, bool through_compatible) const
    {
        std::vector<char> r(n_, 0);
        for (int x = 0; x < n_; x++) {
            if (set[x]) {
                r[x] = 1;
                continue;
            }
            if (through_compatible && !compat_[x]) continue;
            for (int a : p_.items[x].args)
                if (r[a]) {
                    r[x] = 1;
                    break;
                }
        }
        return r;
    }

private:
    const Plan &p_;
    const int n_;
    std::vector<char> compat_;
};

static int count_outputs(const Plan &p, const std::vector<char> &set)
{
    int k = 0;
    for (size_t i = 0; i < set.size(); i++) k += set[i] && p.items[i].output;
    return k;
}

static void output_regions(Plan &p)
{
    const int n = (int)p.items.size();
    for (int root = n - 1; root >= 0; root--) {
        const Item &ri = p.items[root];
        if (!ri.output || ri.region >= 0 || ri.kind != IT_ELEM ||
            (ri.t->dtype != PT_FLOAT32 && ri.t->dtype != PT_FLOAT64))
            continue;
        const RegionBuilder rb(p, root);
        std::vector<char> region(n, 0);
        int cost = 0;
        if (!rb.absorb(root, region, cost) || !region[root]) continue;
        // grow: sweeps over the outputs in item order until one adds nothing
        bool changed = true;
        while (changed) {
            changed = false;
            for (int o = 0; o < n; o++) {
                if (!p.items[o].output || region[o]) continue;
                if (!rb.reaching(region, true)[o]) continue;
                std::vector<char> grown = region;
                int grown_cost = cost;
                if (!rb.absorb(o, grown, grown_cost) || count_outputs(p, grown) > 4) continue;
                region.swap(grown);
                cost = grown_cost;
                changed = true;
            }
        }
        // validate: values that leave, and no way out and back in
        const std::vector<char> back = rb.reaching(region, false);
        std::vector<char> leaves(n, 0);
        bool closed = true;
        for (int x = 0; x < n; x++) {
            if (region[x] && p.items[x].output) leaves[x] = 1;
            for (int a : p.items[x].args) {
                if (!region[x] && region[a]) leaves[a] = 1;
                if (region[x] && !region[a] && back[a]) closed = false;
            }
        }
        int leaving = 0;
        for (int x = 0; x < n; x++) leaving += leaves[x];
        if (!closed || count_outputs(p, region) < 2 || leaving > 4) continue;
        for (int x = 0; x < n; x++) {
            if (!region[x]) continue;
            Item &m = p.items[x];
            m.region = root;
            m.cut = leaves[x] != 0;
            if (m.cut && !m.output) m.reason = "dependent-outputs";
        }
    }
}

// ------------------------------------------------------------ plan build
// ------------------------------------------------------------ row chains
// Short rows make short kernels: a step over [4096, 10] values moves 160 KiB
// and its time is the launch and the first loads of what the step before it
// has just written.  A run of such steps (a softmax cross-entropy and its
// backward: row max, shift, exp, row sums, log, the max's gradient shared
// among ties) is executed by one kernel that gives each row a wave and runs
// the steps one after the other inside it, each step's stores visible to
// the next after a workgroup barrier.  Each fused step evaluates the same
// node functions as its own kernel; each reduction adds in the order of the
// native row kernel for that row length (k_row_reduce with one wave per
// row: each lane folds its elements in index order, four-element chunks
// when the row length is a multiple of 4, then the wave's DPP tree), so the
// chain's values are bit-identical to the steps run one by one.

// Longest row (elements) a chain takes: at most four values per lane, and
// the native reduction of such a row runs one wave per row.
static constexpr long long kChainRowMax = 256;

static bool row_chains_enabled()
{
    // PT_FUSION_ROW_CHAINS=0 runs every step by itself (a tuning and test
    // knob, read once from the environment)
    static const bool on = [] {
        const char *e = getenv("PT_FUSION_ROW_CHAINS");
        return !(e && e[0] == '0');
    }();
    return on;
}

// How kernel `k` reads its leaves relative to its output rows.  A leaf
// reached only through index maps that send output row r into row r of the
// leaf (equal shapes, broadcasts that keep the leading row dimension,
// reshapes that keep the row-major order) gets RL_ROW; any other path adds
// RL_OTHER.
enum { RL_ROW = 1, RL_OTHER = 2 };

static void row_reads(const Plan &p, const Kernel &k, int id, int state, long long rows, std::map<int, int> &leaf,
                      std::set<std::pair<int, int>> &seen)
{
    if (!seen.insert({id, state}).second) return;
    if (is_leaf(p, k, id)) {
        leaf[id] |= state;
        return;
    }
    const Item &it = p.items[id];
    const Tensor &t = *it.t;
    const FusionNode &n = *t.node;
    for (int a : it.args) {
        const Tensor &c = *p.items[a].t;
        int cs = RL_OTHER;
        if (state == RL_ROW) {
            if (n.kind == N_VIEW) {
                // source index = offset + sum coord_d * view_stride_d.  It
                // stays in the row when the view's leading dimension is the
                // rows, one view row steps one source row, and the other
                // dimensions reach less than a source row (reshapes to
                // [rows, 1], broadcasts of [rows, 1] to [rows, n]); or when
                // the view keeps the row-major order (offset 0, the view
                // shape's contiguous strides).
                const size_t total = c.numel();
                bool row = t.ndims >= 1 && t.shape[0] == rows && total % (size_t)rows == 0 &&
                           n.view_offset == 0 && n.view_strides[0] == total / (size_t)rows;
                size_t reach = 0;
                for (int d = 1; d < t.ndims && row; d++) {
                    if (t.shape[d] <= 1) continue;
                    if (n.view_strides[d] >= total) row = false;
                    else reach += (size_t)(t.shape[d] - 1) * n.view_strides[d];
                }
                row = row && reach < total / (size_t)rows;
                size_t cst[kMaxDims];
                contiguous_strides(t.shape, t.ndims, cst);
                bool same = n.view_offset == 0 && total == t.numel();
                for (int d = 0; d < t.ndims && same; d++)
                    if (t.shape[d] > 1 && n.view_strides[d] != cst[d]) same = false;
                if (row || same) cs = RL_ROW;
            } else {
                const bool eq = c.ndims == t.ndims && std::equal(c.shape, c.shape + c.ndims, t.shape);
                const bool lead = c.ndims == t.ndims && t.shape[0] == rows && c.shape[0] == rows;
                if (eq || lead) cs = RL_ROW;
            }
        }
        row_reads(p, k, a, cs, rows, leaf, seen);
    }
}

// Rows of a fused step that may join a chain (0: it may not).
static long long kernel_rows(const Kernel &k)
{
    if (k.ndims < 1 || k.total == 0) return 0;
    const long long rows = k.shape[0];
    if (rows < 2 || rows > 0x7fffffffLL || (long long)k.total / rows > kChainRowMax) return 0;
    return rows;
}

// A native step that may join a chain: a float32 sum / mean / max / min /
// product over the last axis of a materialized [rows, n] float32 value.
static bool chain_reduction(const Plan &p, const Step &st, long long &rows, long long &n)
{
    const Item &it = p.items[st.item];
    const NativeSpec &ns = it.t->node->native;
    if (ns.kind != NAT_REDUCE || it.args.size() != 1 || it.t->dtype != PT_FLOAT32) return false;
    if (ns.op != PT_OP_REDUCE_SUM && ns.op != PT_OP_REDUCE_MEAN && ns.op != PT_OP_REDUCE_MAX &&
        ns.op != PT_OP_REDUCE_MIN && ns.op != PT_OP_REDUCE_PROD)
        return false;
    const Item &a = p.items[it.args[0]];
    if (!(a.kind == IT_NATIVE || (a.kind == IT_ELEM && a.cut))) return false;
    const Tensor &x = *a.t;
    if (x.dtype != PT_FLOAT32 || x.ndims != 2 || ns.axis != 1) return false;
    rows = x.shape[0];
    n = x.shape[1];
    return rows >= 2 && rows <= 0x7fffffffLL && n >= 1 && n <= kChainRowMax;
}

static void emit_row_chain(Plan &p, const RowChain &ch, std::ostringstream &os)
{
    for (int m : ch.members)
        if (!p.steps[m].native) emit_node_functions(p, p.kernels[p.steps[m].kernel], os);
    // no __restrict__: a member reads what an earlier member wrote, through
    // another parameter
    std::string params;
    auto param = [&](const std::string &decl) { params += (params.empty() ? "" : ",") + decl; };
    for (size_t j = 0; j < ch.members.size(); j++) {
        const Step &st = p.steps[ch.members[j]];
        const std::string m = "m" + std::to_string(j);
        if (st.native) {
            param("const void* " + m + "_x");
            param("void* " + m + "_o0");
        } else {
            const Kernel &k = p.kernels[st.kernel];
            for (size_t l = 0; l < k.leaves.size(); l++) param("const void* " + m + "_p" + std::to_string(l));
            for (size_t r = 0; r < k.roots.size(); r++) param("void* " + m + "_o" + std::to_string(r));
        }
    }
    os << "extern \"C\" __global__ __launch_bounds__(64) void " << ch.name << "(" << params << "){\n"
       << "const unsigned lane=threadIdx.x;\nconst unsigned long long row=blockIdx.x;\n";
    for (size_t j = 0; j < ch.members.size(); j++) {
        const Step &st = p.steps[ch.members[j]];
        const std::string m = "m" + std::to_string(j);
        if (st.native) {
            long long rows = 0, n = 0;
            chain_reduction(p, st, rows, n);
            const int op = p.items[st.item].t->node->native.op;
            const char *f = op == PT_OP_REDUCE_MAX ? "pt_rc_max" : op == PT_OP_REDUCE_MIN ? "pt_rc_min"
                          : op == PT_OP_REDUCE_PROD ? "pt_rc_mul" : "pt_rc_add";
            const char *ident = op == PT_OP_REDUCE_MAX ? "-__builtin_inff()" : op == PT_OP_REDUCE_MIN ? "__builtin_inff()"
                              : op == PT_OP_REDUCE_PROD ? "1.0f" : "0.0f";
            os << "{const float* x=static_cast<const float*>(" << m << "_x)+row*" << n << "ULL;\nfloat a=" << ident
               << ";\n";
            if (ch.vec4[j])
                os << "for(unsigned e=4u*lane;e<" << n << "u;e+=256u){a=" << f << "(a,x[e]);a=" << f << "(a,x[e+1]);a="
                   << f << "(a,x[e+2]);a=" << f << "(a,x[e+3]);}\n";
            else
                os << "for(unsigned e=lane;e<" << n << "u;e+=64u)a=" << f << "(a,x[e]);\n";
            os << "a=pt_rc_wave(a," << f << ");\n";
            if (op == PT_OP_REDUCE_MEAN) os << "a=a/(float)" << n << ";\n";
            os << "if(lane==0)static_cast<float*>(" << m << "_o0)[row]=a;}\n";
        } else {
            const Kernel &k = p.kernels[st.kernel];
            const long long n = (long long)k.total / ch.rows;
            std::string args;
            for (size_t l = 0; l < k.leaves.size(); l++) args += m + "_p" + std::to_string(l) + ",";
            os << "for(unsigned long long e=lane;e<" << n << "ULL;e+=64ULL){\nconst unsigned long long i=row*" << n
               << "ULL+e;\n";
            for (size_t r = 0; r < k.roots.size(); r++) {
                const Tensor &t = *p.items[k.roots[r]].t;
                os << "static_cast<" << storage_type(t.dtype) << "*>(" << m << "_o" << r << ")[i]="
                   << store_conv(t.dtype, k.name + "_n" + std::to_string(k.roots[r]) + "(" + args + "i)") << ";\n";
            }
            os << "}\n";
        }
        if (j + 1 < ch.members.size()) os << "__syncthreads();\n";
    }
    os << "}\n";
}

static void find_row_chains(Plan &p)
{
    const int ns = (int)p.steps.size();
    p.step_chain.assign(ns, -1);
    if (!row_chains_enabled() || ns < 2) return;
    const int nitems = (int)p.items.size();
    std::vector<int> producer(nitems, -1);
    for (int i = 0; i < ns; i++) {
        const Step &st = p.steps[i];
        if (st.native) producer[st.item] = i;
        else
            for (int r : p.kernels[st.kernel].roots) producer[r] = i;
    }
    // rows of step i as a member of a chain whose steps are marked in
    // `in_chain` (0: it cannot join); a fused step must read every value
    // the chain produces within the row
    auto member_rows = [&](int i, const std::vector<char> &in_chain, char &vec4) -> long long {
        const Step &st = p.steps[i];
        vec4 = 0;
        if (st.native) {
            long long rows = 0, n = 0;
            if (!chain_reduction(p, st, rows, n)) return 0;
            // the native row kernel reads 16-byte chunks of such rows
            vec4 = n % 4 == 0;
            return rows;
        }
        const Kernel &k = p.kernels[st.kernel];
        const long long rows = kernel_rows(k);
        if (!rows) return 0;
        std::map<int, int> leaf;
        std::set<std::pair<int, int>> seen;
        for (int r : k.roots) row_reads(p, k, r, RL_ROW, rows, leaf, seen);
        for (const auto &e : leaf) {
            const int pr = producer[e.first];
            if (pr >= 0 && in_chain[pr] && e.second != RL_ROW) return 0;
        }
        return rows;
    };
    // A chain is a run of consecutive steps: the plan's order, and the
    // branch each step runs on, stay as they are, with the run collapsed
    // into one launch at its last step.
    int next_free = 0;
    for (int s0 = 0; s0 < ns; s0++) {
        if (s0 < next_free) continue;
        std::vector<char> in_chain(ns, 0);
        char v4 = 0;
        const long long rows = member_rows(s0, in_chain, v4);
        if (!rows) continue;
        RowChain ch;
        ch.rows = rows;
        ch.members = {s0};
        ch.vec4 = {v4};
        in_chain[s0] = 1;
        for (int j = s0 + 1; j < ns && member_rows(j, in_chain, v4) == rows; j++) {
            ch.members.push_back(j);
            ch.vec4.push_back(v4);
            in_chain[j] = 1;
        }
        if (ch.members.size() < 2) continue;
        const int c = (int)p.chains.size();
        ch.name = "rc" + std::to_string(c);
        for (int m : ch.members) p.step_chain[m] = c;
        next_free = ch.members.back() + 1;
        p.chains.push_back(ch);
    }
    if (p.chains.empty()) return;
    std::ostringstream os;
    emit_prelude(os);
    // the native row kernel's wave reduction (wave_all in pt_common.h): DPP
    // quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror,
    // then lanes 0 + 16 and 32 + 48
    os << "__device__ __forceinline__ float pt_rc_add(float a,float b){return a+b;}\n"
          "__device__ __forceinline__ float pt_rc_mul(float a,float b){return a*b;}\n"
          "__device__ __forceinline__ float pt_rc_max(float a,float b){return fmaxf(a,b);}\n"
          "__device__ __forceinline__ float pt_rc_min(float a,float b){return fminf(a,b);}\n"
          "template<typename F>__device__ __forceinline__ float pt_rc_wave(float v,F f){\n"
          "v=f(v,__uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0,(int)__float_as_uint(v),0xB1,0xF,0xF,false)));\n"
          "v=f(v,__uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0,(int)__float_as_uint(v),0x4E,0xF,0xF,false)));\n"
          "v=f(v,__uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0,(int)__float_as_uint(v),0x141,0xF,0xF,false)));\n"
          "v=f(v,__uint_as_float((unsigned)__builtin_amdgcn_update_dpp(0,(int)__float_as_uint(v),0x140,0xF,0xF,false)));\n"
          "const int iv=(int)__float_as_uint(v);\n"
          "const float a=__uint_as_float((unsigned)__builtin_amdgcn_readlane(iv,0));\n"
          "const float b=__uint_as_float((unsigned)__builtin_amdgcn_readlane(iv,16));\n"
          "const float c=__uint_as_float((unsigned)__builtin_amdgcn_readlane(iv,32));\n"
          "const float d=__uint_as_float((unsigned)__builtin_amdgcn_readlane(iv,48));\n"
          "return f(f(a,b),f(c,d));}\n";
    for (const RowChain &ch : p.chains) emit_row_chain(p, ch, os);
    p.chain_source = os.str();
}

static Plan *build_plan(const std::vector<TensorP> &roots, const std::vector<TensorP> &inputs)
{
    auto *p = new Plan();
    p->input_examples = inputs;
    std::map<const Tensor *, int> index;
    for (const TensorP &r : roots) {
        int id = collect(*p, r, index);
        p->items[id].output = true;
        p->outputs.push_back(id);
    }
    for (int id : p->outputs)
        if (p->items[id].kind == IT_ELEM) p->items[id].cut = true;
    output_regions(*p);
    // Schedule by levels (as soon as possible).  A native step runs one
    // level after the kernels it reads (at the level of natives it reads);
    // a materialized elementwise root runs one level after kernel roots of
    // another shape that it reads, at the level of natives it reads, and at
    // the level of same-shape roots it reads, which it then evaluates
    // inline in the same kernel (the vector kernel evaluates each node once
    // per element; the general kernel's node functions recompute, so inline
    // chains are at most kMaxInline deep).  Each level runs its natives in
    // item order, then one kernel per shape (at most kMaxRoots roots each).
    // at most 4 outputs per fused step: the reference's region output
    // budget (fusion_plan.c:352, 381)
    constexpr size_t kMaxRoots = 4;
    constexpr int kMaxInline = 2;
    const int nitems = (int)p->items.size();
    std::vector<int> level(nitems, -1), depth(nitems, 0);
    auto same_shape = [&](int a, int b) {
        const Tensor &x = *p->items[a].t, &y = *p->items[b].t;
        return x.ndims == y.ndims && std::equal(x.shape, x.shape + x.ndims, y.shape);
    };
    int max_level = 0;
    // outputs already placed, by (level, shape representative): a value cut
    // for expression cost is evaluated inline only by an output that joins
    // other outputs of its shape (a dependent-output group, as the
    // reference's regions); otherwise its consumers read it back, which is
    // what the cost budget is for
    std::vector<std::pair<int, int>> placed_outputs;
    auto outputs_at = [&](int L, int id) {
        int n = 0;
        for (auto &po : placed_outputs)
            if (po.first == L && same_shape(po.second, id)) n++;
        return n;
    };
    auto inlinable = [&](int d, int id) {
        if (p->items[d].kind != IT_ELEM || !same_shape(d, id)) return false;
        const Item &di = p->items[d];
        if (di.reason && !strcmp(di.reason, "expression-cost"))
            return p->items[id].output && outputs_at(level[d], id) >= 1;
        return true;
    };
    // A root may read a root of another shape placed at its own level: the
    // level's kernels then run that shape first (as the reference schedules
    // a region's cut dependencies before it, fusion_plan.c:104-122).  These
    // orderings are edges between shape groups of one level and must stay
    // acyclic; a root that would close a cycle moves one level down.
    struct Order { int level, before, after; };
    std::vector<Order> orders;
    auto precedes = [&](int L, int from, int to) {
        std::vector<int> stack = {from}, seen;
        while (!stack.empty()) {
            int x = stack.back();
            stack.pop_back();
            if (same_shape(x, to)) return true;
            bool visited = false;
            for (int s : seen) visited = visited || same_shape(s, x);
            if (visited) continue;
            seen.push_back(x);
            for (const Order &o : orders)
                if (o.level == L && same_shape(o.before, x)) stack.push_back(o.after);
        }
        return false;
    };
    auto cross = [&](int d, int id) {
        return p->items[id].kind == IT_ELEM && p->items[d].kind == IT_ELEM && !same_shape(d, id);
    };
    for (int id = 0; id < nitems; id++) {
        Item &it = p->items[id];
        if (it.kind != IT_NATIVE && !(it.kind == IT_ELEM && it.cut)) continue;
        std::vector<int> deps;
        direct_deps(*p, id, deps);
        int L = 0;
        for (int d : deps) {
            bool dn = p->items[d].kind == IT_NATIVE;
            bool in_line = it.kind == IT_ELEM && !dn && inlinable(d, id);
            L = std::max(L, level[d] + (dn || in_line || cross(d, id) ? 0 : 1));
        }
        for (int d : deps)
            if (cross(d, id) && level[d] == L && precedes(L, id, d)) {
                L++;
                break;
            }
        int dp = 0;
        if (it.kind == IT_ELEM)
            for (int d : deps)
                if (level[d] == L && inlinable(d, id)) dp = std::max(dp, depth[d] + 1);
        if (dp > kMaxInline) {
            L++;
            dp = 0;
        }
        level[id] = L;
        depth[id] = dp;
        max_level = std::max(max_level, L);
        for (int d : deps)
            if (cross(d, id) && level[d] == L) orders.push_back({L, d, id});
        if (it.kind == IT_ELEM && it.output) placed_outputs.push_back({L, id});
    }
    std::vector<std::vector<int>> users(nitems);
    for (int id = 0; id < nitems; id++)
        for (int a : p->items[id].args) users[a].push_back(id);
    for (int L = 0; L <= max_level; L++) {
        for (int id = 0; id < nitems; id++)
            if (level[id] == L && p->items[id].kind == IT_NATIVE) {
                Step st;
                st.native = true;
                st.item = id;
                p->steps.push_back(st);
            }
        // roots of this level by shape, in item order
        std::vector<std::vector<int>> groups;
        for (int id = 0; id < nitems; id++) {
            if (level[id] != L || p->items[id].kind != IT_ELEM) continue;
            std::vector<int> *g = nullptr;
            for (auto &c : groups)
                if (same_shape(c[0], id)) g = &c;
            if (!g) {
                groups.emplace_back();
                g = &groups.back();
            }
            g->push_back(id);
        }
        // shape groups in an order that honours this level's orderings
        // (stable: first appearance among the groups that are free to run)
        std::vector<std::vector<int>> ordered;
        while (!groups.empty()) {
            size_t pick = 0;
            for (size_t c = 0; c < groups.size(); c++) {
                bool ready = true;
                for (const Order &o : orders)
                    if (o.level == L && same_shape(o.after, groups[c][0]))
                        for (size_t e = 0; e < groups.size(); e++)
                            if (e != c && same_shape(o.before, groups[e][0])) ready = false;
                if (ready) {
                    pick = c;
                    break;
                }
            }
            ordered.push_back(groups[pick]);
            groups.erase(groups.begin() + (long)pick);
        }
        groups.swap(ordered);
        std::vector<Kernel> ks;
        for (auto &g : groups) {
            // A root cut only for expression cost whose every use lies in
            // this group is evaluated inline by its users instead of being
            // written out (as the reference's dependent-output regions keep
            // their members uncut, fusion_plan.c:381-389).
            std::vector<int> kept;
            int group_outputs = 0;
            for (int a : g) group_outputs += p->items[a].output ? 1 : 0;
            for (int a : g) {
                Item &it = p->items[a];
                bool inline_it = group_outputs >= 2 && !it.output && it.reason &&
                                 !strcmp(it.reason, "expression-cost");
                if (inline_it) {
                    std::vector<int> stack = {a};
                    std::vector<char> seen(nitems, 0);
                    while (!stack.empty() && inline_it) {
                        int x = stack.back();
                        stack.pop_back();
                        for (int u : users[x]) {
                            if (seen[u]) continue;
                            seen[u] = 1;
                            const Item &ui = p->items[u];
                            if (ui.kind != IT_ELEM) inline_it = false;
                            else if (!ui.cut) stack.push_back(u);
                            else if (std::find(g.begin(), g.end(), u) == g.end()) inline_it = false;
                        }
                    }
                }
                if (inline_it) it.cut = false;
                else kept.push_back(a);
            }
            // at most kMaxRoots roots per kernel, in order; the roots of one
            // region stay together
            std::vector<std::vector<int>> chunks(1);
            std::vector<char> placed(kept.size(), 0);
            for (size_t a = 0; a < kept.size(); a++) {
                if (placed[a]) continue;
                std::vector<int> unit;
                const int reg = p->items[kept[a]].region;
                for (size_t b2 = a; b2 < kept.size(); b2++)
                    if (!placed[b2] && (b2 == a || (reg >= 0 && p->items[kept[b2]].region == reg))) {
                        unit.push_back(kept[b2]);
                        placed[b2] = 1;
                    }
                if (chunks.back().size() + unit.size() > kMaxRoots && !chunks.back().empty())
                    chunks.emplace_back();
                chunks.back().insert(chunks.back().end(), unit.begin(), unit.end());
            }
            for (const std::vector<int> &chunk : chunks) {
                if (chunk.empty()) continue;
                Kernel k;
                const Tensor &t = *p->items[chunk[0]].t;
                k.ndims = t.ndims;
                for (int d = 0; d < t.ndims; d++) k.shape[d] = t.shape[d];
                k.total = t.numel();
                k.roots = chunk;
                int outs = 0;
                for (int r : k.roots) outs += p->items[r].output ? 1 : 0;
                // A kernel of two or more outputs is a dependent-output group
                // when a root reads another root, or two roots evaluate a
                // common same-shape node inline (the reference's regions join
                // outputs connected through shared members,
                // fusion_plan.c:288-301, 337-358).
                std::vector<int> owner(nitems, -1);
                for (size_t ri = 0; ri < k.roots.size() && outs >= 2 && !k.dependent; ri++) {
                    const int r = k.roots[ri];
                    std::vector<int> stack(p->items[r].args.begin(), p->items[r].args.end());
                    std::vector<char> seen(nitems, 0);
                    while (!stack.empty() && !k.dependent) {
                        int x = stack.back();
                        stack.pop_back();
                        if (seen[x]) continue;
                        seen[x] = 1;
                        if (std::find(k.roots.begin(), k.roots.end(), x) != k.roots.end()) {
                            k.dependent = true;
                            break;
                        }
                        const Item &xi = p->items[x];
                        if (xi.kind != IT_ELEM || xi.cut || !same_shape(x, r)) continue;
                        if (owner[x] >= 0 && owner[x] != (int)ri) k.dependent = true;
                        owner[x] = (int)ri;
                        for (int a : xi.args) stack.push_back(a);
                    }
                }
                ks.push_back(k);
            }
        }
        for (Kernel &k : ks) {
            k.name = "fk" + std::to_string(p->kernels.size());
            Step st;
            st.kernel = (int)p->kernels.size();
            p->kernels.push_back(k);
            p->steps.push_back(st);
        }
    }
    // leaves, maps and source
    std::ostringstream os;
    emit_prelude(os);
    for (Kernel &k : p->kernels) {
        bool affine = true;
        std::vector<std::pair<int, CoordMap>> uses;
        for (int r : k.roots) gather(*p, k, r, identity_map(k.ndims), affine, uses);
        // a leaf used through two different maps keeps the general path
        k.leaf_maps.assign(k.leaves.size(), LeafMap());
        std::vector<bool> seen(k.leaves.size(), false);
        for (auto &u : uses) {
            int slot = (int)(std::find(k.leaves.begin(), k.leaves.end(), u.first) - k.leaves.begin());
            const Item &it = p->items[u.first];
            const Tensor &src = it.kind == IT_INPUT ? *p->input_examples[it.input_index] : *it.t;
            bool own = it.kind == IT_CONST || it.kind == IT_INPUT;
            size_t cstr[kMaxDims];
            contiguous_strides(it.t->shape, it.t->ndims, cstr);
            LeafMap m;
            m.affine = true;
            for (int kk = 0; kk < u.second.nd_item; kk++) {
                long long s = own ? (long long)src.strides[kk] : (long long)cstr[kk];
                m.offset += u.second.base[kk] * s;
                for (int d = 0; d < k.ndims; d++) m.stride[d] += u.second.coef[kk][d] * s;
            }
            if (seen[slot] && memcmp(&k.leaf_maps[slot], &m, sizeof(m)) != 0) affine = false;
            k.leaf_maps[slot] = m;
            seen[slot] = true;
        }
        k.affine = affine && k.ndims > 0 && k.total % 4 == 0 && k.shape[k.ndims - 1] % 4 == 0;
        k.leaf_vec.assign(k.leaves.size(), false);
        k.leaf_stream.assign(k.leaves.size(), false);
        if (k.affine) {
            for (size_t l = 0; l < k.leaves.size(); l++) {
                const LeafMap &m = k.leaf_maps[l];
                const Tensor &lt = *p->items[k.leaves[l]].t;
                size_t es = dtype_size(lt.dtype);
                bool v = m.stride[k.ndims - 1] == 1 && (es == 4 || es == 2) && m.offset % 4 == 0;
                for (int d = 0; d < k.ndims - 1 && v; d++) v = m.stride[d] % 4 == 0;
                k.leaf_vec[l] = v;
                // a leaf that advances along every output dimension of
                // extent > 1 is read exactly once per element
                bool stream = true;
                for (int d = 0; d < k.ndims; d++)
                    if (k.shape[d] > 1 && m.stride[d] == 0) stream = false;
                k.leaf_stream[l] = stream;
            }
            emit_vector(*p, k, os);
        }
        emit_general(*p, k, os);
    }
    p->source = os.str();
    // graph compatibility: every step can be captured except indexed native
    // steps, whose validation is read back on the host after each execution
    for (const Step &st : p->steps) {
        if (!st.native) continue;
        const int kind = p->items[st.item].t->node->native.kind;
        if (kind == NAT_GATHER || kind == NAT_SCATTER_ADD) p->indexed = true;
    }
    // (fusion_plan.c:505-509: an indexed step makes the plan neither stream-
    // nor graph-compatible, with the incompatibility "indexed-operation")
    if (p->indexed) {
        p->graph_compatible = false;
        p->incompatibility = "indexed-operation";
    }
    find_row_chains(*p);
    return p;
}

// ------------------------------------------------------------ execution
static uint64_t now_ns()
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

// Storage for item `id` (materialized elementwise root): reuse the cached
// buffer when nobody else holds it any more.
static std::shared_ptr<Storage> buffer_for(Plan &p, int id, size_t bytes)
{
    auto it = p.cache.find(id);
    if (it != p.cache.end() && it->second.use_count() == 1 && it->second->bytes >= bytes) {
        p.buffer_reuses++;
        return it->second;
    }
    auto st = std::make_shared<Storage>();
    st->bytes = bytes;
    if (!check_status(pt_alloc(&st->ptr, bytes ? bytes : 1, nullptr), "Fusion buffer allocation"))
        return nullptr;
    p.tensor_allocations++;
    p.cache[id] = st;
    return st;
}

static const void *leaf_ptr(const Plan &p, const std::vector<TensorP> &vals, int id)
{
    const TensorP &v = vals[id];
    (void)p;
    return v->data();
}

static bool launch_kernel(Plan &p, Kernel &k, std::vector<TensorP> &vals)
{
    std::vector<void *> ptrs;
    bool vec_ok = k.affine && k.fn_vec;
    for (size_t l = 0; l < k.leaves.size(); l++) {
        const void *ptr = leaf_ptr(p, vals, k.leaves[l]);
        ptrs.push_back(const_cast<void *>(ptr));
        if (k.leaf_vec[l] && ((uintptr_t)ptr & 15)) vec_ok = false;
    }
    for (int r : k.roots) {
        void *ptr = vals[r]->data();
        ptrs.push_back(ptr);
        if ((uintptr_t)ptr & 15) vec_ok = false;
    }
    if (!k.total) return true;
    std::vector<void *> params;
    for (void *&ptr : ptrs) params.push_back(&ptr);
    size_t work = vec_ok ? k.total / 4 : k.total;
    // one thread per work item: a full grid streams HBM faster on gfx950
    // than a capped grid-stride loop (the loop remains for grids above the
    // hardware limit)
    size_t blocks = (work + 255) / 256;
    if (blocks > 0x7fffffffu) blocks = 0x7fffffffu;
    return check_status(pt_launch(vec_ok ? k.fn_vec : k.fn_scalar, (unsigned)blocks, 256, params.data(),
                                  nullptr),
                        "Fusion kernel launch failed");
}

// Operand of a native step: a materialized value, or an uncut chain of
// views over one, passed as a strided view of the value's storage.
static TensorP native_arg(const Plan &p, std::vector<TensorP> &vals, int id)
{
    const Item &it = p.items[id];
    if (it.kind != IT_ELEM || it.cut || it.t->node->kind != N_VIEW) return vals[id];
    TensorP src = native_arg(p, vals, it.args[0]);
    if (!src) return nullptr;
    if (!src->contiguous()) src = materialize(src);
    if (!src) return nullptr;
    const FusionNode &n = *it.t->node;
    TensorP v = make_meta(it.t->shape, it.t->ndims, it.t->dtype);
    if (!v) return nullptr;
    v->storage = src->storage;
    v->offset = src->offset + n.view_offset;
    for (int d = 0; d < v->ndims; d++) v->strides[d] = n.view_strides[d];
    v->read_only = true;
    return v;
}

// One step on the current stream.
static bool run_step(Plan &p, const Step &st, std::vector<TensorP> &vals)
{
    if (!st.native) return launch_kernel(p, p.kernels[st.kernel], vals);
    Item &it = p.items[st.item];
    std::vector<TensorP> ins;
    for (int a : it.args) {
        TensorP v = native_arg(p, vals, a);
        if (!v) return false;
        ins.push_back(v);
    }
    preset_output(vals[st.item]);
    TensorP out = native_execute(it.t->node->native, ins);
    preset_output(nullptr);
    if (!out) return false;
    vals[st.item] = out;
    return true;
}

// The chain's kernel: one 64-thread workgroup per row.  A reduction whose
// chunked order was assumed needs its rows 16-byte aligned, as the native
// kernel does to read them in chunks; otherwise `launched` stays false.
static bool launch_chain(Plan &p, RowChain &ch, std::vector<TensorP> &vals, bool &launched)
{
    launched = false;
    std::vector<void *> ptrs;
    for (size_t j = 0; j < ch.members.size(); j++) {
        const Step &st = p.steps[ch.members[j]];
        if (st.native) {
            TensorP x = native_arg(p, vals, p.items[st.item].args[0]);
            if (!x) return false;
            const void *xp = x->data();
            if (ch.vec4[j] && ((uintptr_t)xp & 15u)) return true;
            ptrs.push_back(const_cast<void *>(xp));
            ptrs.push_back(vals[st.item]->data());
        } else {
            const Kernel &k = p.kernels[st.kernel];
            for (int l : k.leaves) ptrs.push_back(const_cast<void *>(leaf_ptr(p, vals, l)));
            for (int r : k.roots) ptrs.push_back(vals[r]->data());
        }
    }
    std::vector<void *> params;
    for (void *&q : ptrs) params.push_back(&q);
    launched = true;
    return check_status(pt_launch(ch.fn, (unsigned)ch.rows, 64, params.data(), nullptr),
                        "Fusion row-chain launch failed");
}

// A chain at the position of its last member: its kernel, or its members
// one by one (no chain kernel, or rows it cannot take).
static bool run_chain(Plan &p, int c, std::vector<TensorP> &vals)
{
    RowChain &ch = p.chains[c];
    bool launched = false;
    if (ch.fn && !launch_chain(p, ch, vals, launched)) return false;
    if (launched) return true;
    p.chain_fallbacks++;
    for (int m : ch.members)
        if (!run_step(p, p.steps[m], vals)) return false;
    return true;
}

// Chain of step i, or -1.
static int chain_of(const Plan &p, int i) { return p.step_chain.empty() ? -1 : p.step_chain[i]; }

static bool run_steps(Plan &p, std::vector<TensorP> &vals)
{
    for (int i = 0; i < (int)p.steps.size(); i++) {
        const int c = chain_of(p, i);
        if (c >= 0) {
            if (i == p.chains[c].members.back() && !run_chain(p, c, vals)) return false;
            continue;
        }
        if (!run_step(p, p.steps[i], vals)) return false;
    }
    return true;
}

// Graph capture over several streams.  Each step runs on a branch, after
// waiting on the events of the steps it reads that ran on other branches.
// Independent steps (the weight and input gradients of one layer, a
// bias-gradient reduction beside a GEMM, the optimizer update of one layer
// beside the next layer's products) then become parallel branches of the
// captured graph, as the reference's plan stream orders native and fused
// steps (fusion_execute.c:385-412); the values and the order of every
// dependency are unchanged.  The branch is chosen on estimated times (a
// list schedule): the one where the step could start first, preferring the
// branch of its latest dependency when that branch has not moved on (no
// cross-branch wait), then the least recently used one.  A product that
// fills the device queues behind the previous such product whatever its
// branch, so a short step is not placed behind a product it does not need:
// in the config-5 step the first layer's bias-gradient sum and its update
// ran after the second layer's weight gradient on one branch, 19 us after
// the last product.
static constexpr int kBranches = 3;

// Rough duration of a step in microseconds, for branch placement only:
// products at 120 TFLOP/s, other steps at 6 TB/s of what they read and
// write, plus 3 us per launch.  `heavy`: a product of at least 2 GFLOP,
// which holds every CU while it runs.
static double step_cost_us(const Plan &p, const Step &st, bool &heavy)
{
    heavy = false;
    auto bytes_of = [&](int id) {
        const TensorP &t = p.items[id].t;
        return (double)t->numel() * (double)dtype_size(t->dtype);
    };
    if (st.native) {
        const Item &it = p.items[st.item];
        if (it.t->node->native.kind == 0 && it.args.size() == 2) {  // matmul
            const TensorP &a = p.items[it.args[0]].t;
            const double flops = 2.0 * (double)it.t->numel() * (double)a->shape[a->ndims - 1];
            heavy = flops >= 2e9;
            return 3.0 + flops / 120e6;
        }
        double b = bytes_of(st.item);
        for (int a : it.args) b += bytes_of(a);
        return 3.0 + b / 6e6;
    }
    const Kernel &k = p.kernels[st.kernel];
    double b = 0;
    for (int l : k.leaves) b += bytes_of(l);
    for (int r : k.roots) b += bytes_of(r);
    return 3.0 + b / 6e6;
}

// The side streams of the branches (this thread's), created outside any
// graph capture.
static bool branch_streams(std::vector<pt_stream_t> &streams)
{
    static thread_local std::vector<pt_stream_t> side;
    while ((int)side.size() < kBranches - 1) {
        pt_stream_t s = nullptr;
        if (!check_status(pt_stream_create(&s), "Fusion branch stream")) return false;
        side.push_back(s);
    }
    streams = {pt_default_stream()};
    for (pt_stream_t s : side) streams.push_back(s);
    return true;
}

static bool run_steps_branched(Plan &p, std::vector<TensorP> &vals, std::vector<pt_event_t> &events)
{
    const int ns = (int)p.steps.size();
    // a chain member's values are produced where the chain runs: at its
    // last member
    std::vector<int> producer(p.items.size(), -1);
    for (int i = 0; i < ns; i++) {
        const Step &st = p.steps[i];
        const int c = chain_of(p, i);
        const int at = c >= 0 ? p.chains[c].members.back() : i;
        if (st.native) producer[st.item] = at;
        else
            for (int r : p.kernels[st.kernel].roots) producer[r] = at;
    }
    auto source = [&](int id) {
        // an uncut view chain handed to a native reads the item it views
        while (p.items[id].kind == IT_ELEM && !p.items[id].cut && p.items[id].t->node->kind == N_VIEW)
            id = p.items[id].args[0];
        return id;
    };
    std::vector<pt_stream_t> streams;
    if (!branch_streams(streams)) return false;
    auto new_event = [&](pt_event_t &e) {
        if (!check_status(pt_event_create(&e), "Fusion branch event")) return false;
        events.push_back(e);
        return true;
    };
    bool ok = true;
    pt_event_t fork = nullptr;
    ok = new_event(fork) && check_status(pt_event_record(fork, streams[0]), "Fusion branch fork");
    std::vector<int> branch(ns, 0), last(kBranches, -1);
    std::vector<char> joined(kBranches, 0);
    joined[0] = 1;
    std::vector<pt_event_t> done(ns, nullptr);
    // estimated end of each step, of each branch's queued work and of the
    // last device-filling product
    std::vector<double> est_end(ns, 0.0), free_at(kBranches, 0.0);
    double device_free = 0.0;
    for (int i = 0; i < ns && ok; i++) {
        const Step &st = p.steps[i];
        const int chain = chain_of(p, i);
        if (chain >= 0 && i != p.chains[chain].members.back()) continue;
        std::vector<int> deps;
        auto step_deps = [&](const Step &s) {
            if (s.native) {
                for (int a : p.items[s.item].args) deps.push_back(producer[source(a)]);
            } else {
                for (int l : p.kernels[s.kernel].leaves) deps.push_back(producer[l]);
            }
        };
        double cost = 0.0;
        bool heavy = false;
        if (chain >= 0) {
            for (int m : p.chains[chain].members) {
                step_deps(p.steps[m]);
                bool h = false;
                cost += step_cost_us(p, p.steps[m], h);
            }
        } else {
            step_deps(st);
            cost = step_cost_us(p, st, heavy);
        }
        deps.erase(std::remove(deps.begin(), deps.end(), -1), deps.end());
        deps.erase(std::remove(deps.begin(), deps.end(), i), deps.end());
        const int latest = deps.empty() ? -1 : *std::max_element(deps.begin(), deps.end());
        double ready = 0.0;
        for (int d : deps) ready = std::max(ready, est_end[d]);
        const int stay = latest >= 0 && last[branch[latest]] == latest ? branch[latest] : -1;
        auto start_on = [&](int c) {
            const double t = std::max(ready, free_at[c]);
            return heavy ? std::max(t, device_free) : t;
        };
        int b = stay;
        for (int c = 0; c < kBranches; c++) {
            if (b < 0) {
                b = c;
                continue;
            }
            const double sc = start_on(c), sb = start_on(b);
            // earlier start; on a tie keep the dependency's branch, else
            // the least recently used
            if (sc < sb - 1e-9 || (sc <= sb + 1e-9 && b != stay && last[c] < last[b])) b = c;
        }
        est_end[i] = start_on(b) + cost;
        free_at[b] = est_end[i];
        if (heavy) device_free = est_end[i];
        if (!joined[b]) {
            ok = check_status(pt_stream_wait_event(streams[b], fork), "Fusion branch join");
            joined[b] = 1;
        }
        for (int d : deps)
            if (ok && branch[d] != b) ok = check_status(pt_stream_wait_event(streams[b], done[d]), "Fusion branch wait");
        if (!ok) break;
        branch[i] = b;
        last[b] = i;
        pt_stream_set_current(streams[b]);
        ok = chain >= 0 ? run_chain(p, chain, vals) : run_step(p, st, vals);
        pt_stream_set_current(nullptr);
        if (ok) ok = new_event(done[i]) && check_status(pt_event_record(done[i], streams[b]), "Fusion branch event");
    }
    // every branch joins the capture stream again before the capture ends,
    // also after a failure: a capture ended with a side stream still joined
    // to it leaves that stream capturing, and later allocations and frees
    // on the device then fail or crash
    for (int b = 1; b < kBranches; b++) {
        if (!joined[b]) continue;
        pt_event_t e = nullptr;
        const bool joined_ok = new_event(e) && check_status(pt_event_record(e, streams[b]), "Fusion branch end") &&
                               check_status(pt_stream_wait_event(streams[0], e), "Fusion branch end");
        ok = ok && joined_ok;
    }
    return ok;
}

// Allocate materialized values for a run (outside graph capture): kernel
// roots and the outputs of native steps.
static bool prepare_values(Plan &p, std::vector<TensorP> &vals)
{
    auto give = [&](int id) {
        const Tensor &t = *p.items[id].t;
        auto st = buffer_for(p, id, t.numel() * dtype_size(t.dtype));
        if (!st) return false;
        TensorP v = make_meta(t.shape, t.ndims, t.dtype);
        if (!v) return false;
        v->storage = st;
        vals[id] = v;
        return true;
    };
    for (Kernel &k : p.kernels)
        for (int r : k.roots)
            if (!give(r)) return false;
    for (Step &st : p.steps)
        if (st.native && !give(st.item)) return false;
    return true;
}

// First run of a graph plan with native steps: eager, with the natives'
// scratch measured to size the workspace the captured graph will use.
static bool measuring_run(Plan &p, std::vector<TensorP> &vals)
{
    if (!check_status(pt_workspace_begin(nullptr, 0), "Workspace setup failed")) return false;
    bool ok = run_steps(p, vals);
    size_t peak = 0;
    pt_status st = pt_workspace_end(&peak);
    if (!ok) return false;
    if (!check_status(st, "Workspace measurement failed")) return false;
    // at least one granule, so that the arena always has a base
    const size_t bytes = peak > 256 ? peak : 256;
    auto ws = std::make_shared<Storage>();
    ws->bytes = bytes;
    if (!check_status(pt_alloc(&ws->ptr, bytes, nullptr), "Fusion workspace allocation")) return false;
    p.workspace = ws;
    p.tensor_allocations++;
    p.workspace_bytes = bytes;
    p.workspace_sized = true;
    return true;
}

// Record the steps into `p.graph`.  Native steps run with the workspace as
// their scratch and must not allocate; when they cannot (a native that
// needs a temporary copy, scratch beyond the measured peak) the capture is
// dropped, the plan keeps to eager execution and `captured` is false.
static bool capture_steps(Plan &p, std::vector<TensorP> &vals, bool natives, bool &captured)
{
    captured = false;
    std::vector<pt_stream_t> streams;
    if (!branch_streams(streams)) return false;  // before the capture begins
    const uint64_t refusals = allocation_refusals();
    reset_failed_status();
    if (!check_status(pt_graph_begin_capture(nullptr), "Graph capture failed")) return false;
    bool ok = true;
    // branch events stay alive until the capture has ended
    std::vector<pt_event_t> events;
    struct Release {
        std::vector<pt_event_t> &e;
        ~Release()
        {
            for (pt_event_t x : e) pt_event_destroy(x);
        }
    } release{events};
    if (natives)
        ok = check_status(pt_workspace_begin(p.workspace->ptr, p.workspace_bytes), "Workspace setup failed");
    if (ok) {
        allocation_forbidden() = natives;
        ok = run_steps_branched(p, vals, events);
        allocation_forbidden() = false;
        if (natives && !check_status(pt_workspace_end(nullptr), "Workspace release failed")) ok = false;
    }
    if (!ok) {
        pt_stream_set_current(nullptr);
        pt_graph_t scrap = nullptr;
        if (pt_graph_end_capture(nullptr, &scrap) == PT_OK && scrap) pt_graph_destroy(scrap);
        // only a refused allocation (a native that needs a temporary, or
        // scratch beyond the measured workspace) makes the plan eager; any
        // other failure is the caller's error, with its own message
        const bool allocation = allocation_refusals() != refusals || last_failed_status() == PT_ERR_NOMEM;
        if (!allocation) return false;
        p.graph_compatible = false;
        p.incompatibility = "a native step allocates during capture";
        clear_error();
        return true;
    }
    pt_status st = p.graph ? pt_graph_end_capture_update(nullptr, p.graph) : pt_graph_end_capture(nullptr, &p.graph);
    if (!check_status(st, "Graph instantiation failed")) return false;
    captured = true;
    return true;
}

static bool collect_outputs(Plan &p, std::vector<TensorP> &vals, std::vector<TensorP> &outs, uint64_t t0,
                            uint64_t t1);

// Executions of one FusionGraph::replay call that share a graph launch.  The
// GPU leaves a gap of several microseconds between two graph launches on a
// stream and none between kernels inside one graph, so a replay of many
// executions launches a graph that holds this many copies of the steps.
static constexpr int kReplayCopies = 8;

// Capture the steps `copies` times in a row into `p.batch_graph`, for the
// buffers of `p.graph` (plans without native steps: their scratch is handed
// out once per capture).  Each copy forks from and joins the capture stream,
// so copy c + 1 starts after every branch of copy c has ended.
static bool capture_copies(Plan &p, std::vector<TensorP> &vals, int copies)
{
    std::vector<pt_stream_t> streams;
    if (!branch_streams(streams)) return false;  // before the capture begins
    if (p.batch_graph) {
        pt_graph_destroy(p.batch_graph);
        p.batch_graph = nullptr;
        p.batch_ptrs.clear();
    }
    if (!check_status(pt_graph_begin_capture(nullptr), "Graph capture failed")) return false;
    std::vector<pt_event_t> events;
    struct Release {
        std::vector<pt_event_t> &e;
        ~Release()
        {
            for (pt_event_t x : e) pt_event_destroy(x);
        }
    } release{events};
    bool ok = true;
    for (int c = 0; c < copies && ok; c++) ok = run_steps_branched(p, vals, events);
    if (!ok) {
        pt_stream_set_current(nullptr);
        pt_graph_t scrap = nullptr;
        if (pt_graph_end_capture(nullptr, &scrap) == PT_OK && scrap) pt_graph_destroy(scrap);
        return false;
    }
    if (!check_status(pt_graph_end_capture(nullptr, &p.batch_graph), "Graph instantiation failed")) return false;
    p.batch_ptrs = p.graph_ptrs;
    return true;
}

// A plan with indexed native steps: clear the plan's validation record, run
// the steps with the indexed natives recording into it, then read it back
// (the execution's one synchronization) and raise the first invalid index
// as the reference does (fusion_execute.c:755-775).
static bool execute_indexed(Plan &p, std::vector<TensorP> &vals, std::vector<TensorP> &outs, uint64_t t0,
                            uint64_t t1)
{
    if (!p.index_record) {
        auto st = std::make_shared<Storage>();
        if (!check_status(pt_alloc(&st->ptr, 3 * sizeof(int32_t), nullptr), "Fusion index validation buffer"))
            return false;
        st->bytes = 3 * sizeof(int32_t);
        p.index_record = st;
    }
    if (!check_status(pt_memset(p.index_record->ptr, 0, 3 * sizeof(int32_t), nullptr),
                      "Fusion index validation reset"))
        return false;
    index_record() = (int32_t *)p.index_record->ptr;
    bool ok = run_steps(p, vals);
    index_record() = nullptr;
    if (!ok) return false;
    int32_t rec[3] = {0, 0, 0};
    if (!check_status(pt_memcpy_d2h(rec, p.index_record->ptr, sizeof(rec), nullptr),
                      "Fusion index validation synchronization failed"))
        return false;
    p.synchronizations++;
    if (rec[0] == 1) {
        set_invalid("gather indices must be within [0, %d)", rec[2]);
        return false;
    }
    if (rec[0] == 2) {
        set_invalid("scatterAdd indices must be within [0, %d)", rec[2]);
        return false;
    }
    return collect_outputs(p, vals, outs, t0, t1);
}

// `copies` == kReplayCopies (FusionGraph::replay): when the plan runs from
// its captured graph and has no native steps, that many executions run in a
// row on the same buffers through one graph launch.  `*ran_copies` is set to the
// number of executions done (1 otherwise).
static bool execute(Plan &p, const std::vector<TensorP> &inputs, std::vector<TensorP> &outs, bool wait,
                    int copies = 1, int *ran_copies = nullptr)
{
    if (ran_copies) *ran_copies = 1;
    uint64_t t0 = now_ns();
    std::vector<TensorP> vals(p.items.size());
    for (size_t i = 0; i < p.items.size(); i++) {
        Item &it = p.items[i];
        if (it.kind == IT_CONST) {
            if (it.t->lazy() && !fusion_materialize(it.t)) return false;
            vals[i] = it.t;
        } else if (it.kind == IT_INPUT) {
            vals[i] = inputs[it.input_index];
        }
    }
    if (!prepare_values(p, vals)) return false;
    uint64_t t1 = now_ns();
    bool graph_ok = p.use_graph && p.graph_compatible;
    bool native_present = false;
    for (Step &st : p.steps) native_present = native_present || st.native;
    bool ran = false;
    if (graph_ok && native_present && !p.workspace_sized) {
        if (!measuring_run(p, vals)) return false;
        ran = true;
    }
    if (graph_ok && !ran) {
        std::vector<void *> ptrs;
        for (size_t i = 0; i < vals.size(); i++)
            if (vals[i]) ptrs.push_back(vals[i]->data());
        if (!p.graph || ptrs != p.graph_ptrs) {
            // a pending execution may still be running the executable graph
            // that the capture below updates
            if (p.pending && !check_status(pt_stream_synchronize(nullptr), "Fusion synchronization failed"))
                return false;
            bool captured = false;
            if (!capture_steps(p, vals, native_present, captured)) return false;
            if (captured) {
                p.graph_ptrs = ptrs;
            } else {
                if (!run_steps(p, vals)) return false;
                ran = true;
            }
        }
        if (!ran && copies == kReplayCopies && !native_present) {
            if ((!p.batch_graph || p.batch_ptrs != p.graph_ptrs) && !capture_copies(p, vals, copies)) return false;
            if (!check_status(pt_graph_launch(p.batch_graph, nullptr), "Graph launch failed")) return false;
            // graphLaunches counts hipGraphLaunch calls (one per cuGraphLaunch in
            // fusion_execute.c:588-595), executions count executions
            p.graph_launches++;
            p.executions += copies - 1;
            if (ran_copies) *ran_copies = copies;
        } else if (!ran) {
            if (!check_status(pt_graph_launch(p.graph, nullptr), "Graph launch failed")) return false;
            p.graph_launches++;
        }
    } else if (!ran) {
        if (p.indexed) return execute_indexed(p, vals, outs, t0, t1);
        if (!run_steps(p, vals)) return false;
    }
    if (wait) {
        if (!check_status(pt_stream_synchronize(nullptr), "Fusion synchronization failed")) return false;
        p.synchronizations++;
    }
    return collect_outputs(p, vals, outs, t0, t1);
}

static bool collect_outputs(Plan &p, std::vector<TensorP> &vals, std::vector<TensorP> &outs, uint64_t t0,
                            uint64_t t1)
{
    uint64_t t2 = now_ns();
    outs.clear();
    for (int id : p.outputs) {
        TensorP v = vals[id];
        // outputs are views of the value with the output's metadata
        TensorP o = make_meta(p.items[id].t->shape, p.items[id].t->ndims, p.items[id].t->dtype);
        o->storage = v->storage;
        o->offset = v->offset;
        for (int d = 0; d < o->ndims; d++) o->strides[d] = v->strides[d];
        if (p.items[id].kind == IT_CONST || p.items[id].kind == IT_INPUT) o = materialize(v);
        outs.push_back(o);
    }
    p.executions++;
    if (p.profiling) {
        uint64_t t3 = now_ns();
        p.profiled++;
        p.bind_ns += t1 - t0;
        p.execute_ns += t2 - t1;
        p.collect_ns += t3 - t2;
    }
    return true;
}

// Row-chain modules, by source.  Kept apart from the Fusion module cache,
// whose statistics describe the plans' own generated sources; modules stay
// loaded (plans hold their handles), and past kChainModules sources new
// chains compile without being kept.
static std::mutex g_chain_mu;
static std::unordered_map<std::string, pt_module_t> g_chain_modules;
static constexpr size_t kChainModules = 64;

static pt_module_t load_chain_module(const std::string &src)
{
    std::lock_guard<std::mutex> lock(g_chain_mu);
    auto it = g_chain_modules.find(src);
    if (it != g_chain_modules.end()) return it->second;
    pt_module_t m = nullptr;
    static char log[8192];
    if (!check_status(pt_rtc_compile(src.c_str(), "fusion_rows.hip", &m, log, sizeof(log)),
                      "Fusion row-chain compilation failed"))
        return nullptr;
    if (g_chain_modules.size() < kChainModules) g_chain_modules[src] = m;
    return m;
}

static bool compile_plan(Plan &p)
{
    if (!p.kernels.empty()) {
        p.module = load_module(p.source, p.cache_hit);
        if (!p.module) return false;
        for (Kernel &k : p.kernels) {
            if (k.affine && !check_status(pt_module_function(p.module, (k.name + "_v").c_str(), &k.fn_vec),
                                          "Fusion kernel lookup"))
                return false;
            if (!check_status(pt_module_function(p.module, (k.name + "_s").c_str(), &k.fn_scalar),
                              "Fusion kernel lookup"))
                return false;
        }
    }
    if (!p.chains.empty()) {
        p.chain_module = load_chain_module(p.chain_source);
        if (!p.chain_module) return false;
        for (RowChain &ch : p.chains)
            if (!check_status(pt_module_function(p.chain_module, ch.name.c_str(), &ch.fn), "Fusion row-chain lookup"))
                return false;
    }
    return true;
}

bool fusion_materialize(const TensorP &t)
{
    if (t->fusion_failed) {
        set_runtime("Tensor belongs to an aborted Fusion capture");
        return false;
    }
    if (!t->lazy()) return true;
    // evaluate the recorded subgraph producing `t` now (Fusion::run reads
    // inside the callback), then keep `t` as a concrete value
    Scope *saved = t_scope;
    t_scope = nullptr;
    std::unique_ptr<Plan> p(build_plan({t}, saved ? saved->inputs : std::vector<TensorP>()));
    for (const Item &it : p->items)
        if (it.kind == IT_INPUT) {
            t_scope = saved;
            set_runtime("Fusion::compile cannot read tensor data during capture; use FusionGraph::run");
            return false;
        }
    bool ok = compile_plan(*p);
    std::vector<TensorP> outs;
    if (ok) ok = execute(*p, {}, outs, false);
    t_scope = saved;
    if (!ok) return false;
    t->storage = outs[0]->storage;
    t->offset = outs[0]->offset;
    for (int d = 0; d < t->ndims; d++) t->strides[d] = outs[0]->strides[d];
    return true;
}

}  // namespace phpt

// =================================================================== C API
using namespace phpt;

struct phpt_graph {
    Plan *plan;
};

static phpt_tensor *wrap(const TensorP &t)
{
    if (!t) return nullptr;
    auto *h = new phpt_tensor;
    h->t = t;
    return h;
}

static thread_local std::string t_text;

extern "C" {

int phpt_fusion_begin(int compiling)
{
    clear_error();
    if (t_scope) {
        set_runtime("Fusion scopes cannot be nested");
        return -1;
    }
    t_scope = new Scope();
    t_scope->compiling = compiling != 0;
    return 0;
}

int phpt_fusion_active(void) { return fusion_active() ? 1 : 0; }

void phpt_fusion_abort(void)
{
    // values recorded by the aborted callback can never be computed
    // (fusion_failed, fusion.c:160-166)
    if (t_scope)
        for (const TensorP &t : t_scope->recorded)
            if (t->lazy()) t->fusion_failed = true;
    delete t_scope;
    t_scope = nullptr;
}

phpt_tensor *phpt_fusion_input(phpt_tensor *example, int index)
{
    clear_error();
    if (!t_scope) {
        set_invalid("No active Fusion scope");
        return nullptr;
    }
    const TensorP &ex = example->t;
    if (ex->lazy()) {
        set_invalid("Fusion inputs must be materialized CudaArray values");
        return nullptr;
    }
    auto n = std::make_shared<FusionNode>();
    n->kind = N_INPUT;
    n->input_index = index;
    TensorP t = make_meta(ex->shape, ex->ndims, ex->dtype);
    if (!t) return nullptr;
    t->node = n;
    if ((int)t_scope->inputs.size() <= index) t_scope->inputs.resize(index + 1);
    t_scope->inputs[index] = ex;
    t_scope->recorded.push_back(t);
    return wrap(t);
}

phpt_graph *phpt_fusion_end(phpt_tensor **outputs, int count, int use_graph)
{
    clear_error();
    if (!t_scope) {
        set_invalid("No active Fusion scope");
        return nullptr;
    }
    Scope *scope = t_scope;
    t_scope = nullptr;
    std::vector<TensorP> roots;
    for (int i = 0; i < count; i++) roots.push_back(outputs[i]->t);
    Plan *p = build_plan(roots, scope->inputs);
    delete scope;
    p->use_graph = use_graph != 0;
    if (!compile_plan(*p)) {
        delete p;
        return nullptr;
    }
    auto *g = new phpt_graph;
    g->plan = p;
    return g;
}

int phpt_fusion_run_once(phpt_tensor **outputs, int count)
{
    clear_error();
    if (!t_scope) {
        set_invalid("No active Fusion scope");
        return -1;
    }
    Scope *scope = t_scope;
    t_scope = nullptr;
    // roots: the returned values plus recorded values still referenced
    // outside the scope (escaped through closures)
    std::vector<TensorP> roots;
    for (int i = 0; i < count; i++)
        if (outputs[i]->t->lazy()) roots.push_back(outputs[i]->t);
    for (const TensorP &t : scope->recorded)
        if (t->lazy() && t.use_count() > 2 &&
            std::find(roots.begin(), roots.end(), t) == roots.end())
            roots.push_back(t);
    int rc = 0;
    if (!roots.empty()) {
        std::unique_ptr<Plan> p(build_plan(roots, {}));
        std::vector<TensorP> outs;
        if (!compile_plan(*p) || !execute(*p, {}, outs, true)) {
            rc = -1;
        } else {
            for (size_t i = 0; i < roots.size(); i++) {
                roots[i]->storage = outs[i]->storage;
                roots[i]->offset = outs[i]->offset;
                for (int d = 0; d < roots[i]->ndims; d++) roots[i]->strides[d] = outs[i]->strides[d];
                roots[i]->node.reset();
            }
        }
    }
    delete scope;
    return rc;
}

static bool bind(Plan &p, phpt_tensor **inputs, int n, std::vector<TensorP> &out)
{
    if (n != (int)p.input_examples.size()) {
        set_invalid("FusionGraph expects %zu inputs, %d given", p.input_examples.size(), n);
        return false;
    }
    for (int i = 0; i < n; i++) {
        const TensorP &ex = p.input_examples[i];
        const TensorP &t = inputs[i]->t;
        if (t->lazy()) {
            set_invalid("FusionGraph inputs must be materialized");
            return false;
        }
        bool same = t->dtype == ex->dtype && t->ndims == ex->ndims;
        for (int d = 0; same && d < t->ndims; d++)
            same = t->shape[d] == ex->shape[d] && (t->shape[d] == 1 || t->strides[d] == ex->strides[d]);
        if (!same) {
            set_invalid("FusionGraph input %d does not match the captured shape, dtype and strides", i);
            return false;
        }
        out.push_back(t);
    }
    return true;
}

int phpt_graph_run(phpt_graph *g, phpt_tensor **inputs, int ninputs, phpt_tensor **outputs, int noutputs)
{
    clear_error();
    Plan &p = *g->plan;
    std::vector<TensorP> ins, outs;
    if (!bind(p, inputs, ninputs, ins)) return -1;
    if (!execute(p, ins, outs, true)) return -1;
    for (int i = 0; i < noutputs && i < (int)outs.size(); i++) outputs[i] = wrap(outs[i]);
    return (int)outs.size();
}

int phpt_graph_replay(phpt_graph *g, phpt_tensor **inputs, int ninputs, int count, phpt_tensor **outputs,
                      int noutputs)
{
    clear_error();
    Plan &p = *g->plan;
    if (p.pending) {
        set_runtime("FusionGraph has a pending asynchronous replay; wait() first");
        return -1;
    }
    if (count < 1) {
        set_invalid("Replay count must be positive");
        return -1;
    }
    std::vector<TensorP> ins, outs;
    if (!bind(p, inputs, ninputs, ins)) return -1;
    // each execution's outputs are dropped before the next one, so every
    // replay reuses the same buffers and the captured graph; whole groups of
    // kReplayCopies go through one graph launch; one synchronization at the
    // end, after which the last execution's outputs are handed back
    for (int i = 0; i < count;) {
        int ran = 1;
        const int n = count - i >= kReplayCopies ? kReplayCopies : 1;
        outs.clear();
        if (!execute(p, ins, outs, false, n, &ran)) return -1;
        i += ran;
    }
    if (!check_status(pt_stream_synchronize(nullptr), "Fusion synchronization failed")) return -1;
    p.synchronizations++;
    for (int i = 0; i < noutputs && i < (int)outs.size(); i++) outputs[i] = wrap(outs[i]);
    return (int)outs.size();
}

// FusionExecution (fusion.c:561-692): each submitted run owns its outputs,
// the inputs it read and an event recorded after its last step; several may
// be pending at once (they run in submission order on the runtime stream).
struct phpt_execution {
    phpt_graph *graph = nullptr;
    pt_event_t done = nullptr;
    std::vector<TensorP> values;  // outputs, then the retained inputs
    int noutputs = 0;
    bool waited = false;
};

phpt_execution *phpt_graph_run_async(phpt_graph *g, phpt_tensor **inputs, int ninputs)
{
    clear_error();
    Plan &p = *g->plan;
    if (p.indexed) {  // fusion.c:565-569
        set_runtime("runAsync requires a stream-compatible plan: %s", p.incompatibility);
        return nullptr;
    }
    std::vector<TensorP> ins, outs;
    if (!bind(p, inputs, ninputs, ins)) return nullptr;
    if (!execute(p, ins, outs, false)) return nullptr;
    auto *e = new phpt_execution();
    e->graph = g;
    if (!check_status(pt_event_create(&e->done), "event") ||
        !check_status(pt_event_record(e->done, nullptr), "event record")) {
        if (e->done) pt_event_destroy(e->done);
        delete e;
        return nullptr;
    }
    e->noutputs = (int)outs.size();
    e->values = outs;
    for (const TensorP &t : ins) e->values.push_back(t);
    p.pending++;
    return e;
}

int phpt_execution_wait(phpt_execution *e, phpt_tensor **outputs, int noutputs)
{
    clear_error();
    if (!e || e->waited) {
        set_runtime("FusionExecution has no submitted execution");
        return -1;
    }
    if (!check_status(pt_event_synchronize(e->done), "Fusion wait failed")) return -1;
    Plan &p = *e->graph->plan;
    p.synchronizations++;
    p.pending--;
    e->waited = true;
    for (int i = 0; i < noutputs && i < e->noutputs; i++) outputs[i] = wrap(e->values[i]);
    e->values.clear();
    return e->noutputs;
}

int phpt_execution_is_finished(phpt_execution *e)
{
    if (!e || e->waited) return 1;
    int fin = 0;
    if (!check_status(pt_event_query(e->done, &fin), "event query")) return -1;
    return fin;
}

void phpt_execution_release(phpt_execution *e)
{
    if (!e) return;
    if (!e->waited) {
        pt_event_synchronize(e->done);
        e->graph->plan->pending--;
    }
    if (e->done) pt_event_destroy(e->done);
    delete e;
}

int phpt_graph_num_outputs(phpt_graph *g) { return (int)g->plan->outputs.size(); }

const char *phpt_graph_source(phpt_graph *g) { return g->plan->source.c_str(); }

const char *phpt_graph_stats(phpt_graph *g)
{
    Plan &p = *g->plan;
    size_t boundaries = 0, intermediates = 0, aliases = 0;
    for (const Item &it : p.items)
        if (it.alias && !it.cut) aliases++;
    bool native_present = false;
    for (Step &st : p.steps) {
        if (st.native) {
            boundaries++;
            native_present = true;
        }
    }
    for (Kernel &k : p.kernels)
        for (int r : k.roots)
            if (!p.items[r].output) intermediates++;
    std::ostringstream os;
    os << "nodes=" << p.items.size() << ";fusedKernels=" << p.kernels.size() << ";boundaries=" << boundaries
       << ";viewAliases=" << aliases << ";executions=" << p.executions << ";executionSteps=" << p.steps.size() + aliases
       << ";intermediateBuffers=" << intermediates << ";cacheHit=" << (p.cache_hit ? 1 : 0)
       // fusion.c:747-748: a graph only when requested and compatible, else
       // "stream" for stream-compatible plans and "native" for the others
       << ";backend=" << (p.use_graph && p.graph_compatible ? "cuda-graph" : p.indexed ? "native" : "stream")
       << ";asyncCompatible=" << (p.indexed ? 0 : 1) << ";cudaGraphCompatible=" << (p.graph_compatible ? 1 : 0)
       // fusion.c:750-754
       << ";cudaGraphIncompatibility="
       << (p.graph_compatible ? "null" : p.incompatibility ? p.incompatibility : "native-graph-not-supported")
       << ";incompatibility=" << (p.incompatibility ? p.incompatibility : "null")
       << ";graphReplay=" << (p.use_graph && !native_present ? 1 : 0)
       << ";graphLaunches=" << p.graph_launches << ";bufferReuses=" << p.buffer_reuses
       << ";pending=" << p.pending << ";cudaGraphRequested=" << (p.use_graph ? 1 : 0)
       << ";tensorAllocations=" << p.tensor_allocations << ";synchronizations=" << p.synchronizations
       << ";workspaceBuffers=" << p.cache.size() + (p.workspace ? 1 : 0)
       << ";workspaceBytes=" << (p.workspace ? p.workspace_bytes : 0) << ";profiling=" << (p.profiling ? 1 : 0)
       << ";profiledExecutions=" << p.profiled << ";bindTimeNs=" << p.bind_ns
       << ";executeTimeNs=" << p.execute_ns << ";collectTimeNs=" << p.collect_ns << ";";
    // row chains: kernels that each run a run of short-row steps; their
    // members by getPlan step number ("2.3.5/9.10": two chains)
    size_t chained = 0;
    for (const RowChain &ch : p.chains) chained += ch.members.size();
    std::vector<int> number(p.steps.size(), 0);
    {
        int n = 0;
        std::vector<char> shown(p.items.size(), 0);
        for (size_t i = 0; i < p.steps.size(); i++) {
            if (p.steps[i].native)
                for (int a : p.items[p.steps[i].item].args)
                    if (p.items[a].alias && !p.items[a].cut && !shown[a]) {
                        shown[a] = 1;
                        n++;
                    }
            number[i] = n++;
        }
    }
    std::string members;
    for (const RowChain &ch : p.chains) {
        if (!members.empty()) members += "/";
        for (size_t j = 0; j < ch.members.size(); j++)
            members += (j ? "." : "") + std::to_string(number[ch.members[j]]);
    }
    os << "rowChains=" << p.chains.size() << ";rowChainSteps=" << chained << ";rowChainFallbacks=" << p.chain_fallbacks
       << ";rowChainMembers=" << (members.empty() ? "null" : members) << ";";
    t_text = os.str();
    return t_text.c_str();
}

const char *phpt_graph_plan(phpt_graph *g)
{
    Plan &p = *g->plan;
    std::ostringstream os;
    // one entry per step, as FusionGraph::getPlan (fusion.c:775-795):
    // step, root, kind (fused / native), reason, inputs, outputs; plus the
    // generated kernel's name and variant
    int n = 0;
    std::vector<char> shown(p.items.size(), 0);
    for (Step &st : p.steps) {
        if (st.native) {
            static const char *names[] = {"native-matmul", "native-reduction", "native-reduction",
                                          "native-moments", "native-softmax", "native-layernorm",
                                          "native-gather", "native-scatter-add"};
            const Item &it = p.items[st.item];
            // layout aliases: views passed to this native step without a copy
            for (int a : it.args)
                if (p.items[a].alias && !p.items[a].cut && !shown[a]) {
                    shown[a] = 1;
                    os << "step=" << n++ << ",root=" << a << ",kind=view,reason=native-layout-alias,inputs=1,outputs=1;";
                }
            os << "step=" << n << ",root=" << st.item << ",kind=native,reason=" << names[it.t->node->native.kind]
               << ",inputs=" << it.args.size() << ",outputs=1;";
        } else {
            Kernel &k = p.kernels[st.kernel];
            const Item &r0 = p.items[k.roots[0]];
            const char *reason = k.dependent ? "dependent-outputs"
                                 : r0.output  ? "output"
                                 : r0.reason  ? r0.reason
                                              : "dependency";
            os << "step=" << n << ",root=" << k.roots[0] << ",kind=fused,reason=" << reason
               << ",inputs=" << k.leaves.size() << ",outputs=" << k.roots.size() << ",name=" << k.name
               << ",variant=" << (k.affine ? "vector" : "scalar") << ";";
        }
        n++;
    }
    t_text = os.str();
    return t_text.c_str();
}

int phpt_graph_set_profiling(phpt_graph *g, int enabled)
{
    clear_error();
    Plan &p = *g->plan;
    if (p.pending) {
        set_runtime("Cannot change profiling while FusionGraph executions are pending");
        return -1;
    }
    p.profiling = enabled != 0;
    p.profiled = 0;
    p.bind_ns = p.execute_ns = p.collect_ns = 0;
    return 0;
}

void phpt_graph_release(phpt_graph *g)
{
    if (!g) return;
    Plan &p = *g->plan;
    if (p.pending) pt_stream_synchronize(nullptr);
    if (p.graph) pt_graph_destroy(p.graph);
    if (p.batch_graph) pt_graph_destroy(p.batch_graph);
    delete g->plan;
    delete g;
}

const char *phpt_fusion_cache_stats(void)
{
    std::lock_guard<std::mutex> lock(g_cache.mu);
    std::ostringstream os;
    // keys of Fusion::getCacheStats (fusion_cache.c:54-61)
    os << "entries=" << g_cache.modules.size() << ";bytes=" << g_cache.bytes << ";hits=" << g_cache.hits
       << ";misses=" << g_cache.misses << ";compilations=" << g_cache.compilations
       << ";evictions=" << g_cache.evictions << ";maxEntries=" << kCacheEntries << ";maxBytes=" << kCacheBytes
       << ";capacity=" << kCacheEntries << ";";
    t_text = os.str();
    return t_text.c_str();
}

void phpt_fusion_clear_cache(void)
{
    // the cache and its counters start over (fusion_cache_shutdown,
    // fusion_cache.c:41-48); compiled graphs keep their modules
    std::lock_guard<std::mutex> lock(g_cache.mu);
    g_cache.modules.clear();
    g_cache.order.clear();
    g_cache.hits = g_cache.misses = g_cache.evictions = g_cache.compilations = 0;
    g_cache.bytes = 0;
}

}  // extern "C"
