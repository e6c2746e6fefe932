function initstacks_mlp2_ce_b()
    return nothing
end

function mlp2_ce_hv(loss, lossb, x, xb, lab, w1, w1b, b1, b1b, w2, w2b, b2, b2b, h1, h1b, z, zb, i_b, i_in, i_h, i_out, lossd, lossbd, xd, xbd, w1d, w1bd, b1d, b1bd, w2d, w2bd, b2d, b2bd, h1d, h1bd, zd, zbd)
    s1 = 0.0
    s1d = 0.0
    s2 = 0.0
    s2d = 0.0
    se = 0.0
    sed = 0.0
    s1b = 0.0
    s1bd = 0.0
    s2b = 0.0
    s2bd = 0.0
    seb = 0.0
    sebd = 0.0
    for idx = 1:i_b * i_h
        __icse_0 = idx - 1
        i_s = div(__icse_0, i_h) + 1
        i_j = mod(__icse_0, i_h) + 1
        s1d = b1d[i_j]
        s1 = b1[i_j]
        for i_k = 1:i_in
            __icse_1 = (i_k - 1) * i_h + i_j
            __icse_2 = (i_s - 1) * i_in + i_k
            __hcse_3 = x[__icse_2]
            __hcse_4 = w1[__icse_1]
            s1d = s1d + (__hcse_3 * w1d[__icse_1] + __hcse_4 * xd[__icse_2])
            s1 = s1 + __hcse_4 * __hcse_3
        end
        __hcse_5 = tanh(s1)
        __icse_6 = (i_s - 1) * i_h + i_j
        h1d[__icse_6] = (1.0 - __hcse_5 ^ 2) * s1d
        h1[__icse_6] = __hcse_5
    end
    for idx2 = 1:i_b * i_out
        __icse_7 = idx2 - 1
        i_s2 = div(__icse_7, i_out) + 1
        i_o = mod(__icse_7, i_out) + 1
        s2d = b2d[i_o]
        s2 = b2[i_o]
        for i_k2 = 1:i_h
            __icse_8 = (i_k2 - 1) * i_out + i_o
            __icse_9 = (i_s2 - 1) * i_h + i_k2
            __hcse_10 = h1[__icse_9]
            __hcse_11 = w2[__icse_8]
            s2d = s2d + (__hcse_10 * w2d[__icse_8] + __hcse_11 * h1d[__icse_9])
            s2 = s2 + __hcse_11 * __hcse_10
        end
        __icse_12 = (i_s2 - 1) * i_out + i_o
        zd[__icse_12] = s2d
        z[__icse_12] = s2
    end
    for i_s3 = 1:i_b
        sed = 0.0
        se = 0.0
        for i_o2 = 1:i_out
            __icse_13 = (i_s3 - 1) * i_out + i_o2
            __hcse_14 = exp(z[__icse_13])
            sed = sed + __hcse_14 * zd[__icse_13]
            se = se + __hcse_14
        end
        i_l = lab[i_s3]
        __icse_15 = (i_s3 - 1) * i_out + i_l
        lossd[1] = lossd[1] + ((1.0 / se) * sed + -(zd[__icse_15]))
        loss[1] = loss[1] + (log(se) - z[__icse_15])
    end
    for i_s3 = i_b:-1:1
        sed = 0.0
        se = 0.0
        for i_o2 = 1:i_out
            __icse_16 = (i_s3 - 1) * i_out + i_o2
            __hcse_17 = exp(z[__icse_16])
            sed = sed + __hcse_17 * zd[__icse_16]
            se = se + __hcse_17
        end
        i_l = lab[i_s3]
        __hcse_18 = lossb[1]
        __hcse_19 = 1.0 / se
        sebd = sebd + (__hcse_18 * (-(1.0 / se ^ 2) * sed) + __hcse_19 * lossbd[1])
        seb = seb + __hcse_19 * __hcse_18
        __icse_20 = (i_s3 - 1) * i_out + i_l
        zbd[__icse_20] = zbd[__icse_20] + -(lossbd[1])
        zb[__icse_20] = zb[__icse_20] + -__hcse_18
        for i_o2 = i_out:-1:1
            __icse_21 = (i_s3 - 1) * i_out + i_o2
            __hcse_22 = exp(z[__icse_21])
            zbd[__icse_21] = zbd[__icse_21] + (seb * (__hcse_22 * zd[__icse_21]) + __hcse_22 * sebd)
            zb[__icse_21] = zb[__icse_21] + __hcse_22 * seb
        end
        sebd = 0.0
        seb = 0.0
    end
    for idx2 = i_b * i_out:-1:1
        __icse_23 = idx2 - 1
        i_s2 = div(__icse_23, i_out) + 1
        i_o = mod(__icse_23, i_out) + 1
        __icse_24 = (i_s2 - 1) * i_out + i_o
        __oldb_0d = zbd[__icse_24]
        __oldb_0 = zb[__icse_24]
        zbd[__icse_24] = 0.0
        zb[__icse_24] = 0.0
        s2bd = s2bd + __oldb_0d
        s2b = s2b + __oldb_0
        for i_k2 = i_h:-1:1
            __icse_25 = (i_k2 - 1) * i_out + i_o
            __icse_26 = (i_s2 - 1) * i_h + i_k2
            __hcse_27 = h1[__icse_26]
            w2bd[__icse_25] = w2bd[__icse_25] + (s2b * h1d[__icse_26] + __hcse_27 * s2bd)
            w2b[__icse_25] = w2b[__icse_25] + __hcse_27 * s2b
            __hcse_28 = w2[__icse_25]
            h1bd[__icse_26] = h1bd[__icse_26] + (s2b * w2d[__icse_25] + __hcse_28 * s2bd)
            h1b[__icse_26] = h1b[__icse_26] + __hcse_28 * s2b
        end
        __oldb_1d = s2bd
        __oldb_1 = s2b
        s2bd = 0.0
        s2b = 0.0
        b2bd[i_o] = b2bd[i_o] + __oldb_1d
        b2b[i_o] = b2b[i_o] + __oldb_1
    end
    for idx = i_b * i_h:-1:1
        __icse_29 = idx - 1
        i_s = div(__icse_29, i_h) + 1
        i_j = mod(__icse_29, i_h) + 1
        s1d = b1d[i_j]
        s1 = b1[i_j]
        for i_k = 1:i_in
            __icse_30 = (i_k - 1) * i_h + i_j
            __icse_31 = (i_s - 1) * i_in + i_k
            __hcse_32 = x[__icse_31]
            __hcse_33 = w1[__icse_30]
            s1d = s1d + (__hcse_32 * w1d[__icse_30] + __hcse_33 * xd[__icse_31])
            s1 = s1 + __hcse_33 * __hcse_32
        end
        __icse_34 = (i_s - 1) * i_h + i_j
        __oldb_2d = h1bd[__icse_34]
        __oldb_2 = h1b[__icse_34]
        h1bd[__icse_34] = 0.0
        h1b[__icse_34] = 0.0
        __hcse_35 = tanh(s1)
        __hcse_36 = 1.0 - __hcse_35 ^ 2
        s1bd = s1bd + (__oldb_2 * -((2__hcse_35) * (__hcse_36 * s1d)) + __hcse_36 * __oldb_2d)
        s1b = s1b + __hcse_36 * __oldb_2
        for i_k = i_in:-1:1
            __icse_37 = (i_k - 1) * i_h + i_j
            __icse_38 = (i_s - 1) * i_in + i_k
            __hcse_39 = x[__icse_38]
            w1bd[__icse_37] = w1bd[__icse_37] + (s1b * xd[__icse_38] + __hcse_39 * s1bd)
            w1b[__icse_37] = w1b[__icse_37] + __hcse_39 * s1b
            __hcse_40 = w1[__icse_37]
            xbd[__icse_38] = xbd[__icse_38] + (s1b * w1d[__icse_37] + __hcse_40 * s1bd)
            xb[__icse_38] = xb[__icse_38] + __hcse_40 * s1b
        end
        __oldb_3d = s1bd
        __oldb_3 = s1b
        s1bd = 0.0
        s1b = 0.0
        b1bd[i_j] = b1bd[i_j] + __oldb_3d
        b1b[i_j] = b1b[i_j] + __oldb_3
    end
    return nothing
end

function mlp2_ce(loss, x, lab, w1, b1, w2, b2, h1, z, i_b, i_in, i_h, i_out)
    # hidden layer: one iteration per (sample, unit); the feature sum is carried (rule 1)
    for idx = 1:i_b * i_h
        i_s = div(idx - 1, i_h) + 1
        i_j = mod(idx - 1, i_h) + 1
        s1 = b1[i_j]
        for i_k = 1:i_in
            s1 = s1 + w1[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        h1[(i_s - 1) * i_h + i_j] = tanh(s1)
    end
    # output layer: one iteration per (sample, class)
    for idx2 = 1:i_b * i_out
        i_s2 = div(idx2 - 1, i_out) + 1
        i_o = mod(idx2 - 1, i_out) + 1
        s2 = b2[i_o]
        for i_k2 = 1:i_h
            s2 = s2 + w2[(i_k2 - 1) * i_out + i_o] * h1[(i_s2 - 1) * i_h + i_k2]
        end
        z[(i_s2 - 1) * i_out + i_o] = s2
    end
    # softmax cross-entropy of each sample, summed over the batch
    for i_s3 = 1:i_b
        se = 0.0
        for i_o2 = 1:i_out
            se = se + exp(z[(i_s3 - 1) * i_out + i_o2])
        end
        i_l = lab[i_s3]
        loss[1] = loss[1] + (log(se) - z[(i_s3 - 1) * i_out + i_l])
    end
    return nothing
end
