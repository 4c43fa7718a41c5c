// A loaded PtModel run as one native forward (sy_model_*): the library's own
// walk of the YOLOv8 / YOLO11 / YOLO26 detect and segment families,
// channels-last, with the bottleneck shortcuts and concat writes fused into
// the producing convs and the forward captured as a hipGraph from the second
// call of a shape.  This is the path behind the library's benchmarked
// throughput; PtModel.Run over HipBackend's IDeviceBackend members is the
// fallback for every model this class does not recognise.
//
// Mapping.  sy_model_create takes the model's raw tensors (conv weights,
// BatchNorm gamma / beta / running mean / running var, Detect's last-conv
// biases) as one float array in state_dict order, the order
// sy_model_layout lists for a configuration.  The loaded module tree
// (PtModel.cs:84-105) holds exactly those tensors; this class walks it in
// state_dict order (a module's _parameters, then its _buffers, then its
// _modules), skipping what inference never reads: BatchNorm's
// num_batches_tracked, the DFL's fixed weights, training-only branches
// (PtModel.IsTrainingOnly, PtModel.cs:152-153) and the head branches the
// end-to-end mode does not run (PtModel.IsInactiveHeadBranch, :159-164).
// The configuration is inferred (family from the module types, class count,
// reg_max and mask count from the head, BN eps from the first BatchNorm)
// and its scale is the one whose layout every walked tensor matches, shape
// for shape.  A model that matches none is left to PtModel.Run.
//
// Needs one accessor in the reference's PtModel (src/SimdYolo/PtModel.cs):
//     internal PyObject[] Layers => layers;
//
// NOT BUILT IN THIS REPOSITORY (no .NET SDK in the image); source for the
// reference's src/SimdYolo/.
namespace SimdYolo;

internal sealed unsafe class HipWholeModel : IDisposable
{
    // (depth, width, max_channels) per scale n, s, m, l, x: ultralytics
    // yolov8.yaml, and yolo11.yaml / yolo26.yaml (shared).
    private static readonly (float Depth, float Width, int MaxChannels)[] Yolov8Scales =
        [(0.33f, 0.25f, 1024), (0.33f, 0.50f, 1024), (0.67f, 0.75f, 768), (1.00f, 1.00f, 512), (1.00f, 1.25f, 512)];
    private static readonly (float Depth, float Width, int MaxChannels)[] Yolo11Scales =
        [(0.50f, 0.25f, 1024), (0.50f, 0.50f, 1024), (0.50f, 1.00f, 512), (1.00f, 1.00f, 512), (1.00f, 1.50f, 512)];
    private const int ProtoChannels = 256;  // Segment's npr before width scaling in every ultralytics seg yaml

    private readonly nint ctx;
    private nint model;
    private readonly bool segment;

    private HipWholeModel(nint ctx, nint model, bool segment) { this.ctx = ctx; this.model = model; this.segment = segment; }

    public void Dispose()
    {
        if (model != 0) HipNative.ModelDestroy(model);
        model = 0;
    }

    /// <summary>The native forward of <paramref name="pt"/>, or null when its
    /// architecture or tensors match none of the library's configurations.</summary>
    internal static HipWholeModel? TryCreate(nint ctx, PtModel pt)
    {
        PyObject[] layers = pt.Layers;
        if (layers.Length == 0) return null;
        var head = layers[^1];
        bool segment = head.Type.Name is "Segment" or "Segment26";
        if (!segment && head.Type.Name != "Detect") return null;  // pose, OBB, classify, v10: PtModel.Run
        bool endToEnd = ModelInfo.IsEndToEnd(head);
        var types = new HashSet<string>();
        foreach (var layer in layers) CollectTypes(layer, types);
        int arch = endToEnd ? HipNative.ArchYolo26
            : types.Contains("C3k2") ? HipNative.ArchYolo11
            : types.Contains("C2f") ? HipNative.ArchYolov8 : -1;
        if (arch < 0) return null;

        var tensors = new List<Tensor>();
        foreach (var layer in layers) StateDict(layer, tensors);
        float eps = FirstBatchNormEps(layers) ?? 1e-5f;
        var scales = arch == HipNative.ArchYolov8 ? Yolov8Scales : Yolo11Scales;
        foreach (var (depth, width, maxChannels) in scales)
        {
            var cfg = new SyModelConfig
            {
                Arch = arch, Depth = depth, Width = width, MaxChannels = maxChannels,
                Nc = head.Int("nc"), RegMax = head.Int("reg_max", 16), BnEps = eps,
                Nm = segment ? head.Int("nm", 32) : 0, Npr = segment ? ProtoChannels : 0,
            };
            float[]? flat = Flatten(cfg, tensors);
            if (flat is null) continue;
            nint created;
            fixed (float* p = flat) HipNative.Check(HipNative.ModelCreate(ctx, in cfg, p, (nuint)flat.Length, out created));
            return new HipWholeModel(ctx, created, segment);
        }
        return null;
    }

    private static void CollectTypes(PyObject m, HashSet<string> types)
    {
        types.Add(m.Type.Name);
        foreach (var child in m.Children) CollectTypes(child, types);
    }

    private static float? FirstBatchNormEps(IEnumerable<PyObject> modules)
    {
        foreach (var m in modules)
        {
            if (m.Type.Name == "BatchNorm2d") return m.Float("eps", 1e-5f);
            if (FirstBatchNormEps(m.Children) is { } eps) return eps;
        }
        return null;
    }

    // A module's tensors in state_dict order, without what inference never reads.
    private static void StateDict(PyObject m, List<Tensor> into)
    {
        if (m.Type.Name == "DFL") return;  // fixed 0..reg_max-1 weights; the library applies the expectation itself
        foreach (var pair in m.Map("_parameters")) if (pair.Value is Tensor t) into.Add(t);
        foreach (var pair in m.Map("_buffers"))
            if (pair.Value is Tensor t && pair.Key is not "num_batches_tracked") into.Add(t);
        foreach (var pair in m.Map("_modules"))
            if (pair.Value is PyObject child && !Skipped(m, pair.Key)) StateDict(child, into);
    }

    // The rules of PtModel.IsTrainingOnly and PtModel.IsInactiveHeadBranch (PtModel.cs:152-164).
    private static bool Skipped(PyObject module, object key)
    {
        if (module.Type.Name == "Pose26" && key is "flow_model" or "cv4_sigma" or "one2one_cv4_sigma") return true;
        if (module.Type.Name == "Proto26" && key is "semseg") return true;
        if (!module.Has("one2one_cv2") || key is not string name) return false;
        return ModelInfo.IsEndToEnd(module) ? name is "cv2" or "cv3" or "cv4" or "cv4_kpts" : name.StartsWith("one2one_", StringComparison.Ordinal);
    }

    // The tensors as one array in the layout's order, or null if any count or shape differs.
    private static float[]? Flatten(SyModelConfig cfg, List<Tensor> tensors)
    {
        if (HipNative.ModelLayout(in cfg, null, 0, out int count) != 0 || count != tensors.Count) return null;
        var entries = new int[6 * count];
        fixed (int* e = entries)
            if (HipNative.ModelLayout(in cfg, e, count, out _) != 0) return null;
        long total = 0;
        for (int i = 0; i < count; i++)
        {
            int[] dims = [entries[6 * i + 1], entries[6 * i + 2], entries[6 * i + 3], entries[6 * i + 4]];
            if (!SameShape(tensors[i].Shape, dims)) return null;
            total += tensors[i].Length;
        }
        var flat = GC.AllocateUninitializedArray<float>(checked((int)total));
        int offset = 0;
        foreach (var t in tensors)
        {
            t.Data.AsSpan(0, t.Length).CopyTo(flat.AsSpan(offset));
            offset += t.Length;
        }
        return flat;
    }

    // A tensor's shape against a layout entry (d0, d1, d2, d3): equal after
    // padding the tensor's shape with trailing ones (a BatchNorm vector [c]
    // is listed as (c, 1, 1, 1)).
    private static bool SameShape(int[] shape, int[] dims)
    {
        if (shape.Length > 4) return false;
        for (int j = 0; j < 4; j++)
            if ((j < shape.Length ? shape[j] : 1) != dims[j]) return false;
        return true;
    }

    /// <summary>PredictRaw's outputs for one NCHW batch: the head
    /// [B, nc + 4 (+ nm), anchors] (end-to-end models: the selected rows
    /// [B, k, 6 (+ nm)]), and for segment models the prototypes
    /// [B, nm, H / 4, W / 4].  The first call of a shape plans it, tunes its
    /// convolutions and captures the forward; later calls replay the graph.</summary>
    internal Tensor[] Predict(Tensor input, CpuTensorPool? pool)
    {
        if (input.Rank != 4 || input.Shape[1] != 3) throw new ArgumentException("PT YOLO expects NCHW RGB.");
        int batch = input.Shape[0], h = input.Shape[2], w = input.Shape[3];
        HipNative.Check(HipNative.ModelOutputShape(model, batch, h, w, out int d1, out int d2));
        int length = checked(batch * d1 * d2);
        float[] head = pool?.Rent(length, clear: false) ?? GC.AllocateUninitializedArray<float>(length);
        float[] x = input.Data;
        if (!segment)
        {
            fixed (float* src = x)
            fixed (float* dst = head)
                HipNative.Check(HipNative.ModelPredictRaw(model, src, batch, h, w, dst));
            return [new Tensor(head, batch, d1, d2)];
        }
        HipNative.Check(HipNative.ModelProto(model, batch, h, w, out _, out int nm, out int ph, out int pw));
        int protoLength = checked(batch * nm * ph * pw);
        float[] protos = pool?.Rent(protoLength, clear: false) ?? GC.AllocateUninitializedArray<float>(protoLength);
        fixed (float* src = x)
        fixed (float* dst = head)
        fixed (float* pdst = protos)
            HipNative.Check(HipNative.ModelPredictSeg(model, src, batch, h, w, dst, pdst));
        return [new Tensor(head, batch, d1, d2), new Tensor(protos, batch, nm, ph, pw)];
    }
}
